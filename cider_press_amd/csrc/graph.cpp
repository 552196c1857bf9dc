// Runtime node of the quantized-matmul path: a quantized weight leaf, dense
// activation leaves, and lazy QuantizedMatMul / Dequantize nodes evaluated on
// the device's command session.
//
// Mirrors, at the scope of this path only:
//   crates/cider-press-runtime/src/quantized.rs:35-201   QuantizedWeight (+ K padding)
//   crates/cider-press-runtime/src/tensor.rs:2064-2171   Tensor::quantized_matmul
//   crates/cider-press-runtime/src/tensor.rs:1558-1637   Tensor::dequantize_affine
//   crates/cider-press-runtime/src/eval.rs:1293-1394     dispatch_quantized_matmul
//   crates/cider-press-runtime/src/eval.rs:1987-2038     dispatch_dequantize
// The rest of the reference's graph engine (Kahn-wave scheduling, buffer
// pool, barrier elision) is not reproduced: eval walks the node's inputs
// depth-first and encodes each pending node once, in order, on one stream.
#include <memory>
#include <string>
#include <vector>

#include "cpq_internal.hpp"

using cpq::fail;

namespace {

struct DevBuf {
  void* ptr = nullptr;
  size_t len = 0;    // bytes in use
  size_t alloc = 0;  // rounded allocation
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (ptr) (void)hipFree(ptr);
  }
};

struct QWeight {
  cpq_device* dev = nullptr;
  cpq_dtype dtype = CPQ_DTYPE_BF16;
  size_t n = 0, k_physical = 0, k_logical = 0;
  uint32_t bits = 0, group_size = 0;
  DevBuf w, s, b;
};

struct Node {
  enum Kind { Leaf, QuantizedMatMul, Dequantize, EmbedTokens };
  Kind kind = Leaf;
  cpq_device* dev = nullptr;
  cpq_dtype dtype = CPQ_DTYPE_BF16;
  std::vector<size_t> dims;
  DevBuf data;
  bool ready = false;
  std::shared_ptr<Node> x;       // QuantizedMatMul activation / EmbedTokens ids
  std::shared_ptr<QWeight> w;    // QuantizedMatMul / Dequantize / EmbedTokens weight
  size_t numel() const {
    size_t e = 1;
    for (size_t d : dims) e *= d;
    return e;
  }
};

const char* dname(cpq_dtype t) {
  return t == CPQ_DTYPE_BF16 ? "BF16" : t == CPQ_DTYPE_F16 ? "F16" : t == CPQ_DTYPE_U32 ? "U32" : "F32";
}

cpq_status upload_into(cpq_device* dev, DevBuf& buf, const void* host, size_t bytes) {
  cpq_status st = cpq_upload(dev, host, bytes, &buf.ptr, &buf.alloc);
  if (st == CPQ_OK) buf.len = bytes;
  return st;
}

// One lazily created session per device, as the reference keeps one open
// command session per device (commands.rs:46-55); released with the device.
cpq_status session_for(cpq_device* dev, cpq_commands** out) {
  if (!dev->eval_session) {
    cpq_status st = cpq_commands_create(dev, &dev->eval_session);
    if (st != CPQ_OK) return st;
  }
  *out = dev->eval_session;
  return CPQ_OK;
}

cpq_status encode(Node& t, cpq_commands* cmds);

cpq_status encode_inputs(Node& t, cpq_commands* cmds) {
  if (t.x && !t.x->ready) {
    cpq_status st = encode(*t.x, cmds);
    if (st != CPQ_OK) return st;
  }
  return CPQ_OK;
}

cpq_status encode(Node& t, cpq_commands* cmds) {
  if (t.ready) return CPQ_OK;
  cpq_status st = encode_inputs(t, cmds);
  if (st != CPQ_OK) return st;
  const size_t bytes = t.numel() * cpq::dtype_size(t.dtype);
  if (!t.data.ptr) {
    st = cpq_alloc_buffer(t.dev, bytes, &t.data.ptr, &t.data.alloc);
    if (st != CPQ_OK) return st;
    t.data.len = bytes;
  }
  const QWeight& w = *t.w;
  if (t.kind == Node::QuantizedMatMul) {
    // eval.rs:1348-1354: M = product of the activation's leading dims.
    const Node& x = *t.x;
    size_t m = 1;
    for (size_t i = 0; i + 1 < x.dims.size(); ++i) m *= x.dims[i];
    st = cpq_quantized_matmul(cmds, w.dtype, static_cast<const uint32_t*>(w.w.ptr),
                              w.w.len / 4, w.s.ptr, w.s.len / 2, w.b.ptr, w.b.len / 2, x.data.ptr,
                              x.numel(), x.data.alloc, t.data.ptr, m, w.n, w.k_physical,
                              w.group_size, w.bits);
  } else if (t.kind == Node::EmbedTokens) {
    const Node& ids = *t.x;
    st = cpq_embed_tokens(cmds, w.dtype, static_cast<const uint32_t*>(w.w.ptr), w.w.len / 4, w.s.ptr,
                          w.s.len / 2, w.b.ptr, w.b.len / 2, static_cast<const uint32_t*>(ids.data.ptr),
                          ids.numel(), w.n, w.k_physical, t.data.ptr, t.numel(), w.group_size, w.bits);
  } else if (t.kind == Node::Dequantize) {
    st = cpq_affine_dequantize(cmds, w.dtype, static_cast<const uint32_t*>(w.w.ptr), w.w.len / 4,
                               w.s.ptr, w.s.len / 2, w.b.ptr, w.b.len / 2, t.data.ptr, t.numel(),
                               w.group_size, w.bits);
  } else {
    return fail(CPQ_ERR_INVALID_ARGUMENT, "eval: leaf tensor has no data");
  }
  if (st != CPQ_OK) return st;
  t.ready = true;
  return CPQ_OK;
}

}  // namespace

struct cpq_qweight {
  std::shared_ptr<QWeight> p;
};
struct cpq_tensor {
  std::shared_ptr<Node> p;
};

extern "C" {

// quantized.rs:59-125 (from_bytes / from_bytes_k_padded) with the byte-length
// checks of QuantizedWeight::from_bytes_inner.
cpq_status cpq_qweight_from_bytes(cpq_device* dev, cpq_dtype dtype, size_t n, size_t k_physical,
                                  size_t k_logical, uint32_t bits, uint32_t group_size,
                                  const void* weights, size_t weights_bytes, const void* scales,
                                  size_t scales_bytes, const void* biases, size_t biases_bytes,
                                  cpq_qweight** out) {
  if (!dev || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: NULL argument");
  *out = nullptr;
  if (dtype != CPQ_DTYPE_BF16 && dtype != CPQ_DTYPE_F16)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: scales/biases must be BF16 or F16");
  cpq_status st = cpq_quantization_validate(bits, group_size);
  if (st != CPQ_OK) return st;
  if (n == 0 || k_physical == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: shape must be non-empty [N, K]");
  if (k_logical > k_physical)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: k_logical=" + std::to_string(k_logical) +
                                              " > k_physical=" + std::to_string(k_physical));
  if (k_logical % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: k_logical=" + std::to_string(k_logical) +
                                              " must be a multiple of group_size=" +
                                              std::to_string(group_size));
  // Per-row packing (quantized.rs:146-163): K itself, not only N*K, must hold
  // whole groups and whole u32 words.
  if (k_physical % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: inner dim K=" + std::to_string(k_physical) +
                                              " must be a multiple of group_size=" + std::to_string(group_size) +
                                              " (per-row groups must divide evenly)");
  if ((k_physical * bits) % 32 != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: K*bits=" + std::to_string(k_physical * bits) +
                                              " must be a multiple of 32 (per-row packed u32 words must divide "
                                              "evenly)");
  size_t words = 0, groups = 0;
  if (n > SIZE_MAX / k_physical)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: N*K overflows usize");
  st = cpq_packed_word_count(bits, group_size, n * k_physical, &words);
  if (st != CPQ_OK) return st;
  st = cpq_group_count(bits, group_size, n * k_physical, &groups);
  if (st != CPQ_OK) return st;
  if (weights_bytes != words * 4)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: weights byte length " +
                                              std::to_string(weights_bytes) + " != " +
                                              std::to_string(words * 4));
  if (scales_bytes != groups * 2)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: scales byte length " +
                                              std::to_string(scales_bytes) + " != " +
                                              std::to_string(groups * 2));
  if (biases_bytes != groups * 2)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: biases byte length " +
                                              std::to_string(biases_bytes) + " != " +
                                              std::to_string(groups * 2));
  if (!weights || !scales || !biases)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "QuantizedWeight: NULL data");
  auto q = std::make_shared<QWeight>();
  q->dev = dev;
  q->dtype = dtype;
  q->n = n;
  q->k_physical = k_physical;
  q->k_logical = k_logical;
  q->bits = bits;
  q->group_size = group_size;
  if ((st = upload_into(dev, q->w, weights, weights_bytes)) != CPQ_OK) return st;
  if ((st = upload_into(dev, q->s, scales, scales_bytes)) != CPQ_OK) return st;
  if ((st = upload_into(dev, q->b, biases, biases_bytes)) != CPQ_OK) return st;
  *out = new cpq_qweight{q};
  return CPQ_OK;
}

cpq_status cpq_qweight_info(const cpq_qweight* w, size_t* n, size_t* k_physical, size_t* k_logical,
                            uint32_t* bits, uint32_t* group_size, cpq_dtype* dtype) {
  if (!w || !w->p) return fail(CPQ_ERR_INVALID_ARGUMENT, "qweight_info: NULL weight");
  if (n) *n = w->p->n;
  if (k_physical) *k_physical = w->p->k_physical;
  if (k_logical) *k_logical = w->p->k_logical;
  if (bits) *bits = w->p->bits;
  if (group_size) *group_size = w->p->group_size;
  if (dtype) *dtype = w->p->dtype;
  return CPQ_OK;
}

void cpq_qweight_release(cpq_qweight* w) { delete w; }

cpq_status cpq_tensor_from_host(cpq_device* dev, cpq_dtype dtype, const size_t* dims, size_t ndim,
                                const void* data, cpq_tensor** out) {
  if (!dev || !out || (ndim && !dims)) return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor: NULL argument");
  *out = nullptr;
  if (dtype != CPQ_DTYPE_BF16 && dtype != CPQ_DTYPE_F16 && dtype != CPQ_DTYPE_U32)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor: dtype must be BF16, F16 or U32");
  auto t = std::make_shared<Node>();
  t->kind = Node::Leaf;
  t->dev = dev;
  t->dtype = dtype;
  t->dims.assign(dims, dims + ndim);
  const size_t bytes = t->numel() * cpq::dtype_size(dtype);
  if (bytes && !data) return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor: NULL data");
  cpq_status st = upload_into(dev, t->data, data, bytes);
  if (st != CPQ_OK) return st;
  t->ready = true;
  *out = new cpq_tensor{t};
  return CPQ_OK;
}

// tensor.rs:2064-2171
cpq_status cpq_tensor_quantized_matmul(cpq_tensor* x, cpq_qweight* w, int transpose,
                                       cpq_tensor** out) {
  if (!x || !w || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: NULL argument");
  *out = nullptr;
  if (!transpose)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "quantized_matmul: transpose=false direction is not implemented yet "
                "(only the standard `y = x @ W^T` direction is wired)");
  const Node& xa = *x->p;
  const QWeight& q = *w->p;
  if (xa.dev != q.dev)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "quantized_matmul: activation and weight are on different devices");
  if (xa.dtype != q.dtype)
    return fail(CPQ_ERR_INVALID_ARGUMENT, std::string("quantized_matmul: activation must be ") +
                                              dname(q.dtype) + "; got " + dname(xa.dtype));
  if (xa.dims.empty())
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: activation must have rank >= 1");
  const size_t xk = xa.dims.back();
  if (xk != q.k_logical)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: inner dim mismatch: activation last dim " +
                                              std::to_string(xk) + " != weight K " +
                                              std::to_string(q.k_logical));
  size_t m = 1;
  for (size_t i = 0; i + 1 < xa.dims.size(); ++i) m *= xa.dims[i];
  if (m > 1 && q.n % 32 != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "quantized_matmul: weight N (" + std::to_string(q.n) +
                    ") must be a multiple of 32 for the M>1 (prefill) path; only the aligned "
                    "affine_qmm_t variant is wired");
  auto t = std::make_shared<Node>();
  t->kind = Node::QuantizedMatMul;
  t->dev = xa.dev;
  t->dtype = q.dtype;
  t->dims.assign(xa.dims.begin(), xa.dims.end() - 1);
  t->dims.push_back(q.n);
  t->x = x->p;
  t->w = w->p;
  *out = new cpq_tensor{t};
  return CPQ_OK;
}

// tensor.rs:1558-1637
cpq_status cpq_tensor_dequantize(cpq_qweight* w, cpq_tensor** out) {
  if (!w || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "dequantize_affine: NULL argument");
  *out = nullptr;
  const QWeight& q = *w->p;
  auto t = std::make_shared<Node>();
  t->kind = Node::Dequantize;
  t->dev = q.dev;
  t->dtype = q.dtype;
  t->dims = {q.n, q.k_physical};
  t->w = w->p;
  *out = new cpq_tensor{t};
  return CPQ_OK;
}

// nn.rs:123-136 (embed_tokens), with Tensor::gather's index preconditions
// (tensor.rs:1489-1514: dense, rank-1, U32).
cpq_status cpq_tensor_embed_tokens(cpq_tensor* ids, cpq_qweight* w, cpq_tensor** out) {
  if (!ids || !w || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: NULL argument");
  *out = nullptr;
  const Node& x = *ids->p;
  const QWeight& q = *w->p;
  if (x.dev != q.dev) return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: ids and weight are on different devices");
  if (x.dims.size() != 1)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "gather: only rank-1 indices are wired (got rank " +
                                              std::to_string(x.dims.size()) + ")");
  if (x.dtype != CPQ_DTYPE_U32)
    return fail(CPQ_ERR_INVALID_ARGUMENT, std::string("gather: indices must be U32 (got ") + dname(x.dtype) + ")");
  if (q.k_logical != q.k_physical)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: the table must not be K-padded");
  auto t = std::make_shared<Node>();
  t->kind = Node::EmbedTokens;
  t->dev = q.dev;
  t->dtype = q.dtype;
  t->dims = {x.dims[0], q.k_physical};
  t->x = ids->p;
  t->w = w->p;
  *out = new cpq_tensor{t};
  return CPQ_OK;
}

// tensor.rs:2681 (Tensor::eval): encode pending nodes, commit, wait.
cpq_status cpq_tensor_eval(cpq_tensor* t) {
  if (!t) return fail(CPQ_ERR_INVALID_ARGUMENT, "eval: NULL tensor");
  if (t->p->ready) return CPQ_OK;
  cpq_commands* cmds = nullptr;
  cpq_status st = session_for(t->p->dev, &cmds);
  if (st != CPQ_OK) return st;
  st = encode(*t->p, cmds);
  if (st != CPQ_OK) return st;
  return cpq_commands_commit_and_wait(cmds);
}

cpq_status cpq_tensor_shape(cpq_tensor* t, size_t* dims, size_t cap, size_t* ndim) {
  if (!t || !ndim) return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor_shape: NULL argument");
  *ndim = t->p->dims.size();
  for (size_t i = 0; i < t->p->dims.size() && i < cap; ++i) dims[i] = t->p->dims[i];
  return CPQ_OK;
}

cpq_status cpq_tensor_read(cpq_tensor* t, void* host, size_t byte_len) {
  if (!t) return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor_read: NULL tensor");
  if (!t->p->ready)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor_read: tensor has not been evaluated");
  const size_t bytes = t->p->numel() * cpq::dtype_size(t->p->dtype);
  if (byte_len != bytes)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "tensor_read: byte_len " + std::to_string(byte_len) +
                                              " != tensor size " + std::to_string(bytes));
  return cpq_read_buffer(t->p->dev, t->p->data.ptr, host, bytes);
}

void cpq_tensor_release(cpq_tensor* t) { delete t; }

}  // extern "C"
