// Native eager binding of the decode-attention entry points (the package's gqa_decode, gqa_decode_masked and
// gqa_decode_fused without probs) and of the backbone GEMVs (gemv_seg, gemv_resid, gemv_gateup, rmsnorm): the
// argument checks, the output allocation, the device switch, the stream and workspace lookup and the C ABI call in
// one call from Python, as the reference binds its ops with pybind (flash/csrc/bb_attn.cu:462-469,
// flash/csrc/bb_fused.cu:370-377). The attention functions call it first; it returns None when the call needs a
// workspace that does not exist yet, and the Python path then allocates it (outside any graph memory pool),
// registers it here and launches. Every attention check and error message is the Python path's, so both raise the
// same RuntimeError for the same arguments. The GEMVs need no workspace and go through this module alone.
//
// The C ABI functions come as addresses (bind), taken from the library the package has already loaded and checked,
// so this module never loads a second copy of it. Host code only: compiled with g++ against torch's headers.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/hip/HIPFunctions.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/csrc/autograd/python_variable.h>

#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "bz_gemv.h"
#include "bz_gqa_decode.h"

#ifndef BZ_EAGER_BUILD_ID
#define BZ_EAGER_BUILD_ID "unknown"
#endif

namespace {

using DecodeFn = int (*)(const bz_gqa_decode_args*, hipStream_t);
using FusedFn = int (*)(const bz_gqa_decode_fused_args*, hipStream_t);
using StatusFn = const char* (*)(int);
using WsSizeFn = int (*)(int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, size_t*);
using GemvFn = int (*)(const bz_gemv_args*, hipStream_t);
using RmsnormFn = int (*)(const void*, int64_t, const void*, float, void*, int64_t, int32_t, int32_t, hipStream_t);

DecodeFn g_decode = nullptr, g_masked = nullptr, g_noalloc = nullptr;
FusedFn g_fused = nullptr;
StatusFn g_status = nullptr;
WsSizeFn g_ws_size = nullptr;
GemvFn g_gemv = nullptr;
RmsnormFn g_rmsnorm = nullptr;

// (device, raw stream, rows x kv heads) -> the workspace the Python side allocated for that stream
std::map<std::tuple<int, uintptr_t, int64_t>, at::Tensor> g_ws;
// (device or -1, rows, q heads, kv heads, head_dim, capacity, splits, max_seq_len) -> workspace bytes
std::map<std::vector<int64_t>, size_t> g_ws_bytes;

struct Error {
  std::string msg;
};

void check(bool cond, const std::string& msg) {
  if (!cond) throw Error{msg};
}

std::string shape_str(const at::Tensor& t) {  // Python's tuple(t.shape)
  std::string s = "(";
  for (int64_t i = 0; i < t.dim(); ++i) s += (i ? ", " : "") + std::to_string(t.size(i));
  return s + (t.dim() == 1 ? ",)" : ")");
}

const at::Tensor* tensor_or_none(PyObject* o, const char* name) {
  if (o == Py_None) return nullptr;
  if (!THPVariable_Check(o)) throw Error{std::string(name) + " must be a tensor"};
  return &THPVariable_Unpack(o);
}

const at::Tensor& tensor(PyObject* o, const char* name) {
  const at::Tensor* t = tensor_or_none(o, name);
  if (t == nullptr) throw Error{std::string(name) + " must be a tensor"};
  return *t;
}

int combine_code(PyObject* o) {
  if (PyLong_Check(o)) return (int)PyLong_AsLong(o);
  if (PyUnicode_Check(o)) {
    const char* s = PyUnicode_AsUTF8(o);
    if (s && std::string(s) == "auto") return BZ_COMBINE_AUTO;
    if (s && std::string(s) == "last_block") return BZ_COMBINE_LAST_BLOCK;
    if (s && std::string(s) == "kernel") return BZ_COMBINE_KERNEL;
  }
  PyObject* r = PyObject_Repr(o);
  std::string rs = r && PyUnicode_Check(r) ? PyUnicode_AsUTF8(r) : "?";
  Py_XDECREF(r);
  throw Error{"combine must be one of ['auto', 'kernel', 'last_block'], got " + rs};
}

void check_status(int rc, const char* what) {
  if (rc != 0) throw Error{std::string(what) + ": " + (g_status ? g_status(rc) : "error") + " (status " +
                           std::to_string(rc) + ")"};
}

// The checked query/cache/output fields of a call (Python: _check_args with _q_view and _out_view). out: the caller's
// or nullptr; the shape to allocate comes back in out_shape.
void fill_args(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, double scale, const at::Tensor* out,
               int splits, int max_seq_len, int combine, bz_gqa_decode_args& a, std::vector<int64_t>& out_shape) {
  check(q.is_cuda(), "query must be a device tensor");
  check(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 && v.scalar_type() == at::kBFloat16,
        "query, k_cache and v_cache must be bf16");
  check(k.device() == q.device() && v.device() == q.device(), "all tensors must be on one device");
  check(q.dim() >= 1 && q.stride(-1) == 1, "query's head_dim must be contiguous");
  int64_t B, NH, T, D, q_sb, q_sh, q_st;
  if (q.dim() == 4) {
    B = q.size(0), NH = q.size(1), T = q.size(2), D = q.size(3), q_sb = q.stride(0), q_sh = q.stride(1),
    q_st = q.stride(2);
  } else {
    check(q.dim() == 3, "query must be [B, NH, D] or [B, NH, T, D], got shape " + shape_str(q));
    B = q.size(0), NH = q.size(1), T = 1, D = q.size(2), q_sb = q.stride(0), q_sh = q.stride(1), q_st = 0;
  }
  check(k.dim() == 4 && v.sizes() == k.sizes() && v.strides() == k.strides(),
        "k_cache and v_cache must be [B, NKV, capacity, D] with equal shapes and strides");
  check(k.size(0) == B && k.size(3) == D && k.stride(3) == 1,
        "k_cache " + shape_str(k) + " does not match query " + shape_str(q));
  const int64_t NKV = k.size(1), cap = k.size(2);
  int64_t o_sb = 0, o_sh = 0, o_st = 0;
  if (out == nullptr) {
    out_shape = T == 1 ? std::vector<int64_t>{B, NH, D} : std::vector<int64_t>{B, T, NH, D};
    o_sb = T == 1 ? NH * D : T * NH * D;
    o_sh = D;
    o_st = T == 1 ? 0 : NH * D;
  } else {
    const at::Tensor& o = *out;
    check(o.device() == q.device(), "out must be on the query's device");
    check(o.scalar_type() == at::kBFloat16, "out must be bf16");
    check(o.dim() >= 1 && o.stride(-1) == 1, "out's last dimension must be contiguous");
    if (o.dim() == 4 && o.size(0) == B && o.size(1) == T && o.size(2) == NH && o.size(3) == D) {
      o_sb = o.stride(0), o_sh = o.stride(2), o_st = o.stride(1);
    } else if (o.dim() == 4 && o.size(0) == B && o.size(1) == NH && o.size(2) == T && o.size(3) == D) {
      o_sb = o.stride(0), o_sh = o.stride(1), o_st = o.stride(2);
    } else {
      check(T == 1 && o.dim() == 3 && o.size(0) == B && o.size(1) == NH && o.size(2) == D,
            "out must be [B, T, NH, D], [B, NH, T, D] or (T = 1) [B, NH, D] with B=" + std::to_string(B) +
                ", T=" + std::to_string(T) + ", NH=" + std::to_string(NH) + ", D=" + std::to_string(D));
      o_sb = o.stride(0), o_sh = o.stride(1), o_st = 0;
    }
  }
  a = bz_gqa_decode_args{};
  a.q = q.data_ptr();
  a.q_stride_b = q_sb, a.q_stride_h = q_sh;
  a.tokens_per_row = (int32_t)T, a.q_stride_t = q_st, a.out_stride_t = o_st;
  a.k_cache = k.data_ptr(), a.v_cache = v.data_ptr();
  a.kv_stride_b = k.stride(0), a.kv_stride_h = k.stride(1), a.kv_stride_s = k.stride(2);
  a.scale = (float)scale;
  a.out = out ? out->data_ptr() : nullptr;
  a.out_stride_b = o_sb, a.out_stride_h = o_sh;
  a.batch = (int32_t)B, a.num_q_heads = (int32_t)NH, a.num_kv_heads = (int32_t)NKV, a.head_dim = (int32_t)D;
  a.capacity = (int32_t)cap;
  a.num_splits = splits, a.max_seq_len = max_seq_len, a.combine = combine;
}

void int32_rows(const at::Tensor* t, int64_t B, const char* name, const at::Device& dev) {
  check(t != nullptr && t->scalar_type() == at::kInt && t->device() == dev && t->numel() == B && t->is_contiguous(),
        std::string(name) + " must be a contiguous int32 device tensor of " + std::to_string(B) + " elements");
}

void mask_view(const at::Tensor& m, int64_t B, int64_t cap, bz_gqa_decode_args& a, const at::Device& dev) {
  check(m.device() == dev, "mask must be on the query's device");
  check(m.scalar_type() == at::kBFloat16 || m.scalar_type() == at::kFloat, "mask dtype must be bf16 or float32");
  check(m.dim() >= 1 && m.stride(-1) == 1 && m.size(-1) >= cap, "mask's last dim must be contiguous and >= capacity");
  for (int64_t i = 1; i + 1 < m.dim(); ++i) check(m.size(i) == 1, "mask must be [B or 1, 1, 1, S], got " + shape_str(m));
  check(m.size(0) == B || m.size(0) == 1, "mask batch dim must be B or 1");
  a.mask_dtype = m.scalar_type() == at::kBFloat16 ? BZ_MASK_BF16 : BZ_MASK_F32;
  a.mask_stride_b = m.size(0) == 1 ? 0 : m.stride(0);
  a.mask = m.data_ptr();
}

// Makes device idx current for the call and restores the previous one (the Python path's kernels.run_on).
struct DeviceScope {
  c10::DeviceIndex prev, idx;
  explicit DeviceScope(c10::DeviceIndex i) : prev(c10::hip::current_device()), idx(i) {
    if (prev != idx) c10::hip::set_device(idx);
  }
  ~DeviceScope() {
    if (prev != idx) c10::hip::set_device(prev);
  }
};

size_t workspace_bytes(int idx, const bz_gqa_decode_args& a) {
  const int rows = a.batch * (a.tokens_per_row > 1 ? a.tokens_per_row : 1);
  const int dev = a.num_splits == 0 ? idx : -1;  // the default split count depends on the device's CU count
  std::vector<int64_t> key{dev, rows, a.num_q_heads, a.num_kv_heads, a.head_dim, a.capacity, a.num_splits,
                           a.max_seq_len};
  auto it = g_ws_bytes.find(key);
  if (it != g_ws_bytes.end()) return it->second;
  size_t n = 0;
  check_status(g_ws_size(rows, a.num_q_heads, a.num_kv_heads, a.head_dim, a.capacity, a.num_splits, a.max_seq_len,
                         &n),
               "bz_gqa_decode_workspace_size");
  g_ws_bytes.emplace(std::move(key), n);
  return n;
}

// The cached workspace of (device, stream) for these sizes, or nullptr if the Python side has to make one.
const at::Tensor* stream_workspace(int idx, hipStream_t stream, const bz_gqa_decode_args& a) {
  const int64_t groups = (int64_t)a.batch * (a.tokens_per_row > 1 ? a.tokens_per_row : 1) * a.num_kv_heads;
  auto it = g_ws.find({idx, reinterpret_cast<uintptr_t>(stream), groups});
  if (it == g_ws.end()) return nullptr;
  if ((size_t)it->second.numel() < workspace_bytes(idx, a)) return nullptr;
  return &it->second;
}

// Whether the stream is being captured into a graph; a failing query raises, as torch's
// is_current_stream_capturing does (the Python path's check).
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(s, &st);
  if (e != hipSuccess) throw Error{std::string("hipStreamIsCapturing: ") + hipGetErrorString(e)};
  return st == hipStreamCaptureStatusActive;
}

PyObject* result(PyObject* out_obj, const at::Tensor& out) {
  if (out_obj != Py_None) {
    Py_INCREF(out_obj);
    return out_obj;
  }
  return THPVariable_Wrap(out);
}

bool bound() {
  if (g_decode && g_masked && g_noalloc && g_fused && g_status && g_ws_size && g_gemv && g_rmsnorm) return true;
  PyErr_SetString(PyExc_RuntimeError, "_bz_eager: bind() has not been called");
  return false;
}

// decode(q, k_cache, v_cache, seq_lens, kv_start, mask, out, scale, num_splits, max_seq_len, combine, workspace,
//        masked) -> out, or None when the stream has no workspace yet. masked: bz_gqa_decode_masked (the range from
//        the mask; seq_lens and kv_start ignored), else bz_gqa_decode.
PyObject* decode(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!bound()) return nullptr;
  if (nargs != 13) {
    PyErr_SetString(PyExc_TypeError, "decode() takes 13 arguments");
    return nullptr;
  }
  try {
    const at::Tensor& q = tensor(args[0], "query");
    const at::Tensor& k = tensor(args[1], "k_cache");
    const at::Tensor& v = tensor(args[2], "v_cache");
    const at::Tensor* seq_lens = tensor_or_none(args[3], "seq_lens");
    const at::Tensor* kv_start = tensor_or_none(args[4], "kv_start");
    const at::Tensor* mask = tensor_or_none(args[5], "mask");
    const at::Tensor* out = tensor_or_none(args[6], "out");
    const double scale = PyFloat_AsDouble(args[7]);
    const int splits = (int)PyLong_AsLong(args[8]), msl = (int)PyLong_AsLong(args[9]);
    if (PyErr_Occurred()) return nullptr;
    const int comb = combine_code(args[10]);
    const at::Tensor* workspace = tensor_or_none(args[11], "workspace");
    const bool masked = PyObject_IsTrue(args[12]) == 1;
    bz_gqa_decode_args a;
    std::vector<int64_t> out_shape;
    fill_args(q, k, v, scale, out, splits, msl, comb, a, out_shape);
    const at::Device dev = q.device();
    if (masked) {
      check(mask != nullptr, "mask must be a tensor");
      mask_view(*mask, a.batch, a.capacity, a, dev);
    } else {
      int32_rows(seq_lens, a.batch, "seq_lens", dev);
      a.seq_lens = seq_lens->data_ptr<int32_t>();
      if (kv_start) {
        int32_rows(kv_start, a.batch, "kv_start", dev);
        a.kv_start = kv_start->data_ptr<int32_t>();
      }
      if (mask) mask_view(*mask, a.batch, a.capacity, a, dev);
    }
    const int idx = dev.index();
    DeviceScope scope(idx);
    hipStream_t stream = c10::hip::getCurrentHIPStream(idx).stream();
    const bool noalloc = workspace == nullptr && capturing(stream);
    const at::Tensor* ws = workspace;
    if (!noalloc && ws == nullptr) {
      ws = stream_workspace(idx, stream, a);
      if (ws == nullptr) Py_RETURN_NONE;  // the Python path makes the workspace
    }
    at::Tensor out_t = out ? *out : at::empty(out_shape, q.options());
    a.out = out_t.data_ptr();
    if (noalloc) {
      if (masked) a.seq_lens = nullptr, a.kv_start = nullptr;  // the noalloc entry takes the range from the mask
      check_status(g_noalloc(&a, stream), "bz_gqa_decode_noalloc (a call captured without workspace=; pass one for "
                                          "these sizes)");
    } else {
      a.workspace = ws->data_ptr();
      a.workspace_bytes = (size_t)ws->numel() * ws->element_size();
      check_status((masked ? g_masked : g_decode)(&a, stream), masked ? "bz_gqa_decode_masked" : "bz_gqa_decode");
    }
    return result(args[6], out_t);
  } catch (const Error& e) {
    PyErr_SetString(PyExc_RuntimeError, e.msg.c_str());
    return nullptr;
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

// fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out, seq_lens,
//       kv_start, mask, num_splits, max_seq_len, combine, workspace) -> out, or None when the stream has no
//       workspace yet (the Python path then makes one, or raises while the stream is being captured).
PyObject* fused(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!bound()) return nullptr;
  if (nargs != 18) {
    PyErr_SetString(PyExc_TypeError, "fused() takes 18 arguments");
    return nullptr;
  }
  try {
    const at::Tensor& qkv = tensor(args[0], "qkv");
    const at::Tensor& qn = tensor(args[1], "q_norm_weight");
    const at::Tensor& kn = tensor(args[2], "k_norm_weight");
    const double eps = PyFloat_AsDouble(args[3]);
    const at::Tensor& cos = tensor(args[4], "cos");
    const at::Tensor& sin = tensor(args[5], "sin");
    const at::Tensor& k = tensor(args[6], "k_cache");
    const at::Tensor& v = tensor(args[7], "v_cache");
    const at::Tensor& pos = tensor(args[8], "cache_pos");
    const double scale = PyFloat_AsDouble(args[9]);
    const at::Tensor* out = tensor_or_none(args[10], "out");
    const at::Tensor* seq_lens = tensor_or_none(args[11], "seq_lens");
    const at::Tensor* kv_start = tensor_or_none(args[12], "kv_start");
    const at::Tensor* mask = tensor_or_none(args[13], "mask");
    const int splits = (int)PyLong_AsLong(args[14]), msl = (int)PyLong_AsLong(args[15]);
    if (PyErr_Occurred()) return nullptr;
    const int comb = combine_code(args[16]);
    const at::Tensor* workspace = tensor_or_none(args[17], "workspace");
    // the Python path's _fused_args checks, in its order
    check(qkv.dim() == 2 && qkv.stride(1) == 1 && qkv.scalar_type() == at::kBFloat16,
          "qkv must be a bf16 [B, (NH + 2 NKV) * D] tensor with a contiguous last dim");
    check(k.dim() == 4, "k_cache must be [B, NKV, capacity, D]");
    const int64_t B = qkv.size(0), NKV = k.size(1), D = k.size(3);
    const int64_t NH = D > 0 ? qkv.size(1) / D - 2 * NKV : 0;
    check(NH > 0 && qkv.size(1) == (NH + 2 * NKV) * D, "qkv width " + std::to_string(qkv.size(1)) +
                                                           " is not (NH + 2*" + std::to_string(NKV) + ") * " +
                                                           std::to_string(D));
    for (auto [name, w] : {std::pair<const char*, const at::Tensor*>{"q_norm_weight", &qn}, {"k_norm_weight", &kn}})
      check(w->scalar_type() == at::kBFloat16 && w->numel() == D && w->is_contiguous() && w->device() == qkv.device(),
            std::string(name) + " must be a contiguous bf16 [" + std::to_string(D) + "] tensor on the qkv device");
    for (auto [name, t] : {std::pair<const char*, const at::Tensor*>{"cos", &cos}, {"sin", &sin}})
      check(t->scalar_type() == at::kBFloat16 && t->dim() >= 1 && t->stride(-1) == 1 && t->size(0) == B &&
                t->size(-1) == D && t->numel() == B * D && t->device() == qkv.device(),
            std::string(name) + " must be bf16 [B, D] or [B, 1, D]");
    check(cos.stride(0) == sin.stride(0), "cos and sin must share their batch stride");
    check(pos.scalar_type() == at::kLong && pos.numel() >= 1 && pos.device() == qkv.device(),
          "cache_pos must be an int64 device tensor");
    const at::Tensor q_view = qkv.narrow(1, 0, NH * D).view({B, NH, D});
    bz_gqa_decode_fused_args f{};
    std::vector<int64_t> out_shape;
    fill_args(q_view, k, v, scale, out, splits, msl, comb, f.base, out_shape);
    const at::Device dev = qkv.device();
    if (seq_lens) {
      int32_rows(seq_lens, B, "seq_lens", dev);
      f.base.seq_lens = seq_lens->data_ptr<int32_t>();
      if (kv_start) {
        int32_rows(kv_start, B, "kv_start", dev);
        f.base.kv_start = kv_start->data_ptr<int32_t>();
      }
    } else {
      check(mask != nullptr, "gqa_decode_fused needs seq_lens or an interval mask");
    }
    if (mask) {
      check(mask->device() == dev, "mask must be on the qkv device");
      mask_view(*mask, f.base.batch, f.base.capacity, f.base, dev);
    }
    f.qkv = qkv.data_ptr(), f.qkv_stride_b = qkv.stride(0);
    f.q_norm_weight = qn.data_ptr(), f.k_norm_weight = kn.data_ptr(), f.eps = (float)eps;
    f.cos = cos.data_ptr(), f.sin = sin.data_ptr(), f.rope_stride_b = cos.stride(0);
    f.cache_pos = pos.data_ptr<int64_t>();
    const int idx = dev.index();
    DeviceScope scope(idx);
    hipStream_t stream = c10::hip::getCurrentHIPStream(idx).stream();
    const at::Tensor* ws = workspace ? workspace : stream_workspace(idx, stream, f.base);
    if (ws == nullptr) Py_RETURN_NONE;  // the Python path makes the workspace (or raises under capture)
    at::Tensor out_t = out ? *out : at::empty(out_shape, qkv.options());
    f.base.out = out_t.data_ptr();
    f.base.workspace = ws->data_ptr();
    f.base.workspace_bytes = (size_t)ws->numel() * ws->element_size();
    check_status(g_fused(&f, stream), "bz_gqa_decode_fused");
    return result(args[10], out_t);
  } catch (const Error& e) {
    PyErr_SetString(PyExc_RuntimeError, e.msg.c_str());
    return nullptr;
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

// ---- the backbone GEMVs (bz_gemv, bz_rmsnorm)

// x: a bf16 [M, K] device tensor, M 1..4, K and the row stride multiples of 8
void gemv_x(const at::Tensor& x, const char* name, int64_t& M, int64_t& K) {
  check(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.stride(1) == 1,
        std::string(name) + " must be a bf16 [M, K] device tensor with a contiguous last dim");
  M = x.size(0), K = x.size(1);
  check(1 <= M && M <= 4, std::string(name) + ": M must be 1..4, got " + std::to_string(M));
  check(K % 8 == 0 && x.stride(0) % 8 == 0, std::string(name) + ": K and the row stride must be multiples of 8");
}
// a weight: a contiguous bf16 [N, K] device tensor; returns N
int64_t gemv_w(const at::Tensor& w, int64_t K, const char* name) {
  check(w.is_cuda() && w.scalar_type() == at::kBFloat16 && w.is_contiguous() && w.dim() == 2 && w.size(1) == K,
        std::string(name) + " must be a contiguous bf16 [N, " + std::to_string(K) + "] device tensor");
  return w.size(0);
}
// an output or residual: a bf16 [M, N] device tensor with a contiguous last dim
void gemv_y(const at::Tensor& y, int64_t M, int64_t N, const char* name) {
  check(y.is_cuda() && y.scalar_type() == at::kBFloat16 && y.dim() == 2 && y.size(0) == M && y.size(1) == N &&
            y.stride(1) == 1,
        std::string(name) + " must be a bf16 [" + std::to_string(M) + ", " + std::to_string(N) +
            "] device tensor with a contiguous last dim");
}
void gemv_norm_w(const at::Tensor& nw, int64_t K) {
  check(nw.is_cuda() && nw.scalar_type() == at::kBFloat16 && nw.is_contiguous() && nw.numel() == K,
        "the norm weight must be a contiguous bf16 [" + std::to_string(K) + "] device tensor");
}

// gemv(kind, x, norm_weight, eps, w0, w1, w2, res, y) -> y. kind 0: gemv_seg (norm_weight may be None; w1 / w2 None
// or empty for absent segments), 1: gemv_resid (w0, res), 2: gemv_gateup (norm_weight, w0 = gate, w1 = up).
PyObject* gemv(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!bound()) return nullptr;
  if (nargs != 9) {
    PyErr_SetString(PyExc_TypeError, "gemv() takes 9 arguments");
    return nullptr;
  }
  try {
    const long kind = PyLong_AsLong(args[0]);
    const double eps = PyFloat_AsDouble(args[3]);
    if (PyErr_Occurred()) return nullptr;
    const at::Tensor& x = tensor(args[1], "x");
    const at::Tensor* nw = tensor_or_none(args[2], "norm_weight");
    const at::Tensor* w[3] = {tensor_or_none(args[4], "W0"), tensor_or_none(args[5], "W1"),
                              tensor_or_none(args[6], "W2")};
    const at::Tensor* res = tensor_or_none(args[7], "res");
    const at::Tensor& y = tensor(args[8], "y");
    int64_t M, K;
    gemv_x(x, "x", M, K);
    bz_gemv_args a{};
    const char* what;
    if (kind == 0) {
      what = "gemv_seg";
      check(w[0] != nullptr, "W0 must be a tensor");
      const int64_t n0 = gemv_w(*w[0], K, "W0");
      const int64_t n1 = w[1] && w[1]->numel() ? gemv_w(*w[1], K, "W1") : 0;
      const int64_t n2 = w[2] && w[2]->numel() ? gemv_w(*w[2], K, "W2") : 0;
      gemv_y(y, M, n0 + n1 + n2, "y");
      a.epilogue = BZ_GEMV_PLAIN;
      if (nw) {
        gemv_norm_w(*nw, K);
        a.norm_weight = nw->data_ptr(), a.eps = (float)eps;
      }
      a.w[0] = w[0]->data_ptr(), a.n[0] = (int32_t)n0;
      if (n1) a.w[1] = w[1]->data_ptr(), a.n[1] = (int32_t)n1;
      if (n2) a.w[2] = w[2]->data_ptr(), a.n[2] = (int32_t)n2;
    } else if (kind == 1) {
      what = "gemv_resid";
      check(w[0] != nullptr && res != nullptr, "W and res must be tensors");
      const int64_t n = gemv_w(*w[0], K, "W");
      gemv_y(*res, M, n, "res");
      gemv_y(y, M, n, "y");
      a.epilogue = BZ_GEMV_RESIDUAL;
      a.w[0] = w[0]->data_ptr(), a.n[0] = (int32_t)n;
      a.res = res->data_ptr(), a.res_stride = res->stride(0);
    } else if (kind == 2) {
      what = "gemv_gateup";
      check(w[0] != nullptr && w[1] != nullptr && nw != nullptr, "Wg, Wu and the norm weight must be tensors");
      const int64_t n = gemv_w(*w[0], K, "Wg");
      check(gemv_w(*w[1], K, "Wu") == n, "Wg and Wu must have the same number of rows");
      gemv_y(y, M, n, "y");
      gemv_norm_w(*nw, K);
      a.epilogue = BZ_GEMV_SILU_MUL;
      a.norm_weight = nw->data_ptr(), a.eps = (float)eps;
      a.w[0] = w[0]->data_ptr(), a.w[1] = w[1]->data_ptr();
      a.n[0] = (int32_t)n, a.n[1] = (int32_t)n;
    } else {
      throw Error{"gemv: kind must be 0 (seg), 1 (resid) or 2 (gateup)"};
    }
    a.x = x.data_ptr(), a.x_stride = x.stride(0);
    a.y = y.data_ptr(), a.y_stride = y.stride(0);
    a.m = (int32_t)M, a.k = (int32_t)K;
    const int idx = x.device().index();
    DeviceScope scope(idx);
    check_status(g_gemv(&a, c10::hip::getCurrentHIPStream(idx).stream()), what);
    Py_INCREF(args[8]);
    return args[8];
  } catch (const Error& e) {
    PyErr_SetString(PyExc_RuntimeError, e.msg.c_str());
    return nullptr;
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

// rmsnorm(x, w, eps, y) -> y: the standalone row RMSNorm
PyObject* rmsnorm(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!bound()) return nullptr;
  if (nargs != 4) {
    PyErr_SetString(PyExc_TypeError, "rmsnorm() takes 4 arguments");
    return nullptr;
  }
  try {
    const double eps = PyFloat_AsDouble(args[2]);
    if (PyErr_Occurred()) return nullptr;
    const at::Tensor& x = tensor(args[0], "x");
    const at::Tensor& w = tensor(args[1], "w");
    const at::Tensor& y = tensor(args[3], "y");
    check(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.stride(1) == 1,
          "x must be a bf16 [M, K] device tensor with a contiguous last dim");
    const int64_t M = x.size(0), K = x.size(1);
    gemv_norm_w(w, K);
    gemv_y(y, M, K, "y");
    const int idx = x.device().index();
    DeviceScope scope(idx);
    check_status(g_rmsnorm(x.data_ptr(), x.stride(0), w.data_ptr(), (float)eps, y.data_ptr(), y.stride(0),
                           (int32_t)M, (int32_t)K, c10::hip::getCurrentHIPStream(idx).stream()),
                 "rmsnorm");
    Py_INCREF(args[3]);
    return args[3];
  } catch (const Error& e) {
    PyErr_SetString(PyExc_RuntimeError, e.msg.c_str());
    return nullptr;
  } catch (const std::exception& e) {
    PyErr_SetString(PyExc_RuntimeError, e.what());
    return nullptr;
  }
}

// bind(decode, masked, noalloc, fused, status_string, workspace_size, gemv, rmsnorm): the C ABI functions' addresses
PyObject* bind(PyObject*, PyObject* args) {
  unsigned long long d, m, n, f, s, w, g, r;
  if (!PyArg_ParseTuple(args, "KKKKKKKK", &d, &m, &n, &f, &s, &w, &g, &r)) return nullptr;
  g_decode = reinterpret_cast<DecodeFn>(d);
  g_masked = reinterpret_cast<DecodeFn>(m);
  g_noalloc = reinterpret_cast<DecodeFn>(n);
  g_fused = reinterpret_cast<FusedFn>(f);
  g_status = reinterpret_cast<StatusFn>(s);
  g_ws_size = reinterpret_cast<WsSizeFn>(w);
  g_gemv = reinterpret_cast<GemvFn>(g);
  g_rmsnorm = reinterpret_cast<RmsnormFn>(r);
  Py_RETURN_NONE;
}

// register_workspace(device, stream, groups, workspace): the workspace the Python side made for (device, stream)
PyObject* register_workspace(PyObject*, PyObject* args) {
  int idx;
  unsigned long long stream;
  long long groups;
  PyObject* o;
  if (!PyArg_ParseTuple(args, "iKLO", &idx, &stream, &groups, &o)) return nullptr;
  if (!THPVariable_Check(o)) {
    PyErr_SetString(PyExc_TypeError, "register_workspace: a tensor expected");
    return nullptr;
  }
  g_ws[{idx, (uintptr_t)stream, (int64_t)groups}] = THPVariable_Unpack(o);
  Py_RETURN_NONE;
}

PyObject* build_id(PyObject*, PyObject*) { return PyUnicode_FromString(BZ_EAGER_BUILD_ID); }

PyMethodDef kMethods[] = {
    {"decode", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(decode)), METH_FASTCALL,
     "gqa_decode / gqa_decode_masked through the C ABI, or None when the stream has no workspace yet"},
    {"fused", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(fused)), METH_FASTCALL,
     "gqa_decode_fused through the C ABI, or None when the stream has no workspace yet"},
    {"gemv", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(gemv)), METH_FASTCALL,
     "gemv_seg / gemv_resid / gemv_gateup through the C ABI"},
    {"rmsnorm", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(rmsnorm)), METH_FASTCALL,
     "rmsnorm through the C ABI"},
    {"bind", bind, METH_VARARGS, "the C ABI functions' addresses"},
    {"register_workspace", register_workspace, METH_VARARGS, "a workspace made for (device, stream, groups)"},
    {"build_id", build_id, METH_NOARGS, "hash of the sources this module was built from"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_bz_eager",
                       "native eager binding of the decode-attention entries and the backbone GEMVs", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__bz_eager(void) { return PyModule_Create(&kModule); }
