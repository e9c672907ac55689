// Thin torch extension over the C ABI of libint8kv.so (include/int8kv.h): the drop-in operators
// int8_paged_attention, bf16_paged_attention and int8_kv_cache_write called from Python with one
// pybind11 call each, instead of a Python wrapper plus a ctypes call of ~30 marshalled arguments.
//
// What it does per call, and nothing else: the reference's argument checks (raising the same
// exception types: AssertionError for the asserts of src/triton_ops/int8_paged_attention.py:
// 698-719 / int8_cache_write.py:100-115 / bf16_paged_attention.py:118-127, ValueError for an
// unknown impl, :767-768), the output and the decode workspace from torch's caching allocator on
// the input's device, torch's current HIP stream, and one C-ABI call whose strides are the
// tensors' own stride arrays.  No kernel lives here and no state is kept besides the exception
// class the library's status codes are raised as.

#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <cmath>
#include <map>
#include <string>
#include <utility>

#include "int8kv.h"

namespace {

namespace py = pybind11;

struct AssertionFailure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct ValueFailure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct LibraryFailure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

PyObject* g_library_error = PyExc_RuntimeError;  // int8kv._lib.Int8KVError once registered

inline void require(bool ok, const char* what = "") {
  if (!ok) throw AssertionFailure(what);
}

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return INT8KV_F32;
    case at::kHalf: return INT8KV_F16;
    case at::kBFloat16: return INT8KV_BF16;
    case at::kChar: return INT8KV_I8;
    case at::kInt: return INT8KV_I32;
    case at::kLong: return INT8KV_I64;
    default: return -1;
  }
}

const char* status_text(int st) {
  switch (st) {
    case INT8KV_E_NULL: return "INT8KV_E_NULL (a required pointer is NULL)";
    case INT8KV_E_DTYPE: return "INT8KV_E_DTYPE (unsupported element type)";
    case INT8KV_E_SHAPE: return "INT8KV_E_SHAPE (unsupported or inconsistent size)";
    case INT8KV_E_STRIDE: return "INT8KV_E_STRIDE (innermost stride != 1 or rows not 16-byte aligned)";
    case INT8KV_E_WORKSPACE: return "INT8KV_E_WORKSPACE (workspace missing or too small)";
    case INT8KV_E_SCRATCH: return "INT8KV_E_SCRATCH (the call's split partials exceed the library's fixed scratch array)";
    default: return nullptr;
  }
}

void check_status(int st, const char* entry) {
  if (st == 0) return;
  const char* text = status_text(st);
  throw LibraryFailure(std::string(entry) + " failed: " +
                       (text ? std::string(text) : "hipError_t " + std::to_string(st)));
}

bool is_float_source(at::ScalarType t) {
  return t == at::kHalf || t == at::kBFloat16 || t == at::kFloat;
}
bool is_index(at::ScalarType t) { return t == at::kInt || t == at::kLong; }

// 16-byte aligned base and row strides (dims) with a unit innermost stride.
bool rows_aligned16(const at::Tensor& t, std::initializer_list<int> dims) {
  const int64_t e = t.element_size();
  if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 || t.stride(-1) != 1) return false;
  for (int d : dims)
    if ((t.stride(d) * e) % 16) return false;
  return true;
}

// A contiguous copy at a fresh (aligned) address; .contiguous() would keep a misaligned offset.
at::Tensor fresh_copy(const at::Tensor& t) { return t.clone(at::MemoryFormat::Contiguous); }

at::Tensor fp32_vector(const at::Tensor& s) {
  return (s.scalar_type() == at::kFloat && s.is_contiguous()) ? s : s.to(at::kFloat).contiguous();
}

hipStream_t current_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

constexpr int64_t kMaxRanges = 1 << 20;
constexpr int64_t kMaxSplits = 64;  // workgroups per (sequence, kv head) the split merge combines

// The reference's num_splits (src/triton_ops/int8_paged_attention.py:590-604) as the library's
// (num_ranges, flags): none = automatic; 1 = a single pass (one workgroup per sequence and kv
// head, INT8KV_DECODE_PER_SEQUENCE); S >= 2 = S workgroups per sequence and kv head over equal
// shares of its tiles (INT8KV_DECODE_SPLIT_SEQUENCES with num_ranges = S x batch), at most 64.
std::pair<int32_t, uint32_t> split_request(int64_t batch, const c10::optional<int64_t>& num_splits) {
  if (!num_splits.has_value()) return {0, 0u};
  if (*num_splits <= 1) return {0, INT8KV_DECODE_PER_SEQUENCE};
  const int64_t s = std::min<int64_t>(*num_splits, kMaxSplits);
  const int64_t r = std::min<int64_t>(kMaxRanges, s * std::max<int64_t>(1, batch));
  return {(int32_t)r, INT8KV_DECODE_SPLIT_SEQUENCES};
}

// Workspace of an eager call, kept per (device, stream) for the calling host thread: a call's
// partial records are read only by its own merge launch on the same stream, so the next call on
// that stream can reuse the buffer in stream order, while other streams and threads get their
// own.  Saves a caching-allocator round trip per call (~1.3 us of host time on MI355X).  Under
// graph capture it comes from torch's allocator instead (the graph's pool), so a replay never
// shares memory with eager calls.  The tensors are released when the thread ends.
at::Tensor workspace_for(const at::Tensor& like, hipStream_t stream, size_t need) {
  const int64_t bytes = (int64_t)std::max<size_t>(need, 16);
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
    return at::empty({bytes}, like.options().dtype(at::kByte));
  thread_local std::map<std::pair<int, uintptr_t>, at::Tensor> cache;
  at::Tensor& ws = cache[{(int)like.device().index(), reinterpret_cast<uintptr_t>(stream)}];
  if (!ws.defined() || ws.numel() < bytes) ws = at::empty({bytes}, like.options().dtype(at::kByte));
  return ws;
}

// Launches int8kv_paged_decode into `out`; the workspace comes from `workspace` when it is large
// enough, else from workspace_for.
at::Tensor decode_into(at::Tensor query, const at::Tensor& key_cache, const at::Tensor& value_cache,
                       const at::Tensor& block_tables, at::Tensor seq_lens,
                       const c10::optional<at::Tensor>& k_scale,
                       const c10::optional<at::Tensor>& v_scale, at::Tensor out, int64_t num_ranges,
                       int64_t flags, const c10::optional<at::Tensor>& workspace,
                       int64_t min_tiles) {
  const int64_t B = query.size(0), Hq = query.size(1), D = query.size(2);
  if (B == 0) return out;
  const int64_t NB = key_cache.size(0), BS = key_cache.size(1), Hkv = key_cache.size(2);
  if (!rows_aligned16(query, {0, 1})) query = fresh_copy(query);
  if (!seq_lens.is_contiguous()) seq_lens = seq_lens.contiguous();
  const size_t need = int8kv_decode_workspace_bytes((int32_t)Hq, (int32_t)Hkv, (int32_t)D,
                                                    (int32_t)BS, (int32_t)num_ranges);
  const hipStream_t stream = current_stream(query);
  const at::Tensor ws = (workspace.has_value() && (size_t)workspace->numel() >= need)
                            ? *workspace
                            : workspace_for(query, stream, need);
  const int st = int8kv_paged_decode(
      query.data_ptr(), dtype_code(query.scalar_type()), B, (int32_t)Hq, (int32_t)D,
      query.strides().data(), key_cache.data_ptr(), value_cache.data_ptr(),
      dtype_code(key_cache.scalar_type()), NB, (int32_t)BS, (int32_t)Hkv,
      key_cache.strides().data(), value_cache.strides().data(), block_tables.data_ptr(),
      dtype_code(block_tables.scalar_type()), block_tables.size(1), block_tables.strides().data(),
      seq_lens.data_ptr(), dtype_code(seq_lens.scalar_type()),
      k_scale.has_value() ? k_scale->data_ptr<float>() : nullptr,
      v_scale.has_value() ? v_scale->data_ptr<float>() : nullptr, (float)(1.0 / std::sqrt((double)D)),
      out.data_ptr(), out.strides().data(), ws.data_ptr(), (size_t)ws.numel(), (int32_t)num_ranges,
      (int32_t)min_tiles, (uint32_t)flags, stream);
  check_status(st, "int8kv_paged_decode");
  return out;
}

void require_same_device(std::initializer_list<const at::Tensor*> ts, const at::Tensor& first) {
  for (const at::Tensor* t : ts)
    require(t->device() == first.device(), "all tensors must be on one device (the GPU)");
}

// head_dims the decode kernels run (the reference pads any head_dim to a power of two under a
// mask, src/triton_ops/int8_paged_attention.py:556-558,588-589; other sizes fail here, before
// the C ABI, with the reference's AssertionError).
bool head_dim_ok(int64_t d) { return d >= 16 && d <= 256 && d % 16 == 0; }
const char* const kHeadDimText =
    "head_dim must be a multiple of 16 from 16 to 256 (this build's decode kernels)";

// src/triton_ops/int8_paged_attention.py:683-769 (validation :698-719, impl :767-768).
at::Tensor int8_paged_attention(const at::Tensor& query, const at::Tensor& key_cache,
                                const at::Tensor& value_cache, const at::Tensor& block_tables,
                                const at::Tensor& seq_lens, const at::Tensor& k_scale,
                                const at::Tensor& v_scale, bool quantize_q, const std::string& impl,
                                c10::optional<int64_t> num_splits) {
  require(query.dim() == 3 && key_cache.dim() == 4 && value_cache.dim() == 4);
  require(block_tables.dim() == 2 && seq_lens.dim() == 1);
  require(is_float_source(query.scalar_type()));
  require(key_cache.scalar_type() == at::kChar && value_cache.scalar_type() == at::kChar);
  require(is_index(block_tables.scalar_type()) && is_index(seq_lens.scalar_type()));
  const int64_t B = query.size(0), Hq = query.size(1), D = query.size(2);
  const int64_t Hkv = key_cache.size(2);
  require(value_cache.sizes() == key_cache.sizes());
  require(Hkv > 0, "key_cache has no kv heads");
  require(key_cache.size(3) == D && Hq % Hkv == 0);
  require(head_dim_ok(D), kHeadDimText);
  require(block_tables.size(0) == B && seq_lens.numel() == B);
  require(k_scale.dim() == 1 && v_scale.dim() == 1);
  require(k_scale.numel() == Hkv && v_scale.numel() == Hkv);
  require(key_cache.stride(-1) == 1 && value_cache.stride(-1) == 1);
  require(query.is_cuda(), "int8_paged_attention needs GPU tensors");
  require_same_device({&key_cache, &value_cache, &block_tables, &seq_lens, &k_scale, &v_scale},
                      query);
  if (impl != "auto" && impl != "v3" && impl != "v4")
    throw ValueFailure("Unknown impl='" + impl + "'; expected 'auto', 'v3' or 'v4'");
  if (impl == "v3" && !num_splits.has_value()) num_splits = 1;
  at::Tensor out = at::empty({B, Hq, D}, query.options());
  const auto split = split_request(B, num_splits);
  const int64_t flags =
      INT8KV_DECODE_ALL | split.second | (quantize_q ? INT8KV_DECODE_QUANTIZE_Q : 0);
  return decode_into(query, key_cache, value_cache, block_tables, seq_lens, fp32_vector(k_scale),
                     fp32_vector(v_scale), out, split.first, flags, c10::nullopt, 0);
}

// src/triton_ops/bf16_paged_attention.py:118-165.
at::Tensor bf16_paged_attention(const at::Tensor& query, const at::Tensor& key_cache,
                                const at::Tensor& value_cache, const at::Tensor& block_tables,
                                const at::Tensor& seq_lens, c10::optional<int64_t> num_splits) {
  require(query.dim() == 3 && key_cache.dim() == 4 && value_cache.dim() == 4);
  require(block_tables.dim() == 2 && seq_lens.dim() == 1);
  require(is_float_source(query.scalar_type()));
  require(key_cache.scalar_type() == at::kBFloat16 || key_cache.scalar_type() == at::kHalf);
  require(value_cache.scalar_type() == key_cache.scalar_type());
  require(is_index(block_tables.scalar_type()) && is_index(seq_lens.scalar_type()));
  const int64_t B = query.size(0), Hq = query.size(1), D = query.size(2);
  require(value_cache.sizes() == key_cache.sizes());
  require(key_cache.size(2) > 0, "key_cache has no kv heads");
  require(key_cache.size(3) == D && Hq % key_cache.size(2) == 0);
  require(head_dim_ok(D), kHeadDimText);
  require(block_tables.size(0) == B && seq_lens.numel() == B);
  require(key_cache.stride(-1) == 1 && value_cache.stride(-1) == 1);
  require(query.is_cuda(), "bf16_paged_attention needs GPU tensors");
  require_same_device({&key_cache, &value_cache, &block_tables, &seq_lens}, query);
  at::Tensor out = at::empty({B, Hq, D}, query.options());
  const auto split = split_request(B, num_splits);
  return decode_into(query, key_cache, value_cache, block_tables, seq_lens, c10::nullopt,
                     c10::nullopt, out, split.first, INT8KV_DECODE_ALL | split.second,
                     c10::nullopt, 0);
}

// src/triton_ops/int8_cache_write.py:85-149 (validation :100-115).
void int8_kv_cache_write(at::Tensor key, at::Tensor value, const at::Tensor& key_cache,
                         const at::Tensor& value_cache, at::Tensor slot_mapping,
                         const at::Tensor& k_scale, const at::Tensor& v_scale) {
  require(key.dim() == 3 && value.dim() == 3);
  require(key_cache.dim() == 4 && value_cache.dim() == 4);
  require(key.sizes() == value.sizes() && key_cache.sizes() == value_cache.sizes());
  require(key_cache.scalar_type() == at::kChar && value_cache.scalar_type() == at::kChar);
  require(is_float_source(key.scalar_type()) && is_float_source(value.scalar_type()));
  const int64_t T = key.size(0), Hkv = key.size(1), D = key.size(2);
  require(key_cache.size(2) == Hkv && key_cache.size(3) == D);
  require(slot_mapping.dim() == 1 && slot_mapping.numel() == T);
  require(k_scale.dim() == 1 && v_scale.dim() == 1);
  require(k_scale.numel() == Hkv && v_scale.numel() == Hkv);
  require(is_index(slot_mapping.scalar_type()));
  require(key.is_cuda(), "int8_kv_cache_write needs GPU tensors");
  require_same_device({&value, &key_cache, &value_cache, &slot_mapping, &k_scale, &v_scale}, key);
  require(key_cache.stride(-1) == 1 && value_cache.stride(-1) == 1);
  if (T == 0) return;
  if (value.scalar_type() != key.scalar_type()) {
    // One source type per launch; widening to fp32 is exact, so the quotients are unchanged.
    key = key.to(at::kFloat);
    value = value.to(at::kFloat);
  }
  if (!rows_aligned16(key, {0, 1})) key = fresh_copy(key);
  if (!rows_aligned16(value, {0, 1})) value = fresh_copy(value);
  if (!slot_mapping.is_contiguous()) slot_mapping = slot_mapping.contiguous();
  const at::Tensor ks = fp32_vector(k_scale), vs = fp32_vector(v_scale);
  const int st = int8kv_cache_write(
      key.data_ptr(), value.data_ptr(), dtype_code(key.scalar_type()), T, (int32_t)Hkv, (int32_t)D,
      key.strides().data(), value.strides().data(), key_cache.data_ptr(), value_cache.data_ptr(),
      key_cache.size(0), (int32_t)key_cache.size(1), key_cache.strides().data(),
      value_cache.strides().data(), slot_mapping.data_ptr(), dtype_code(slot_mapping.scalar_type()),
      ks.data_ptr<float>(), vs.data_ptr<float>(), current_stream(key));
  check_status(st, "int8kv_cache_write");
}

// The library's decode launcher with caller-chosen ranges/flags/workspace (the decode loop's
// per-layer call, the benchmark's kernel-only timing).
at::Tensor paged_decode(const at::Tensor& query, const at::Tensor& key_cache,
                        const at::Tensor& value_cache, const at::Tensor& block_tables,
                        const at::Tensor& seq_lens, const c10::optional<at::Tensor>& k_scale,
                        const c10::optional<at::Tensor>& v_scale, at::Tensor out, int64_t num_ranges,
                        int64_t flags, const c10::optional<at::Tensor>& workspace, int64_t min_tiles) {
  require(query.dim() == 3 && key_cache.dim() == 4 && value_cache.dim() == 4 &&
          out.sizes() == query.sizes());
  require(block_tables.dim() == 2 && seq_lens.dim() == 1);
  require(value_cache.sizes() == key_cache.sizes());
  require(query.is_cuda(), "paged_decode needs GPU tensors");
  require_same_device({&key_cache, &value_cache, &block_tables, &seq_lens, &out}, query);
  if (k_scale.has_value()) require(k_scale->device() == query.device() && k_scale->dim() == 1);
  if (v_scale.has_value()) require(v_scale->device() == query.device() && v_scale->dim() == 1);
  return decode_into(query, key_cache, value_cache, block_tables, seq_lens, k_scale, v_scale, out,
                     num_ranges, flags, workspace, min_tiles);
}

void set_library_error(py::object cls) {
  cls.inc_ref();  // kept for the life of the process
  g_library_error = cls.ptr();
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const AssertionFailure& e) {
      PyErr_SetString(PyExc_AssertionError, e.what());
    } catch (const ValueFailure& e) {
      PyErr_SetString(PyExc_ValueError, e.what());
    } catch (const LibraryFailure& e) {
      PyErr_SetString(g_library_error, e.what());
    }
  });
  m.def("int8_paged_attention", &int8_paged_attention, py::arg("query"), py::arg("key_cache"),
        py::arg("value_cache"), py::arg("block_tables"), py::arg("seq_lens"), py::arg("k_scale"),
        py::arg("v_scale"), py::arg("quantize_q"), py::arg("impl"), py::arg("num_splits"));
  m.def("bf16_paged_attention", &bf16_paged_attention, py::arg("query"), py::arg("key_cache"),
        py::arg("value_cache"), py::arg("block_tables"), py::arg("seq_lens"), py::arg("num_splits"));
  m.def("int8_kv_cache_write", &int8_kv_cache_write, py::arg("key"), py::arg("value"),
        py::arg("key_cache"), py::arg("value_cache"), py::arg("slot_mapping"), py::arg("k_scale"),
        py::arg("v_scale"));
  m.def("paged_decode", &paged_decode, py::arg("query"), py::arg("key_cache"),
        py::arg("value_cache"), py::arg("block_tables"), py::arg("seq_lens"), py::arg("k_scale"),
        py::arg("v_scale"), py::arg("out"), py::arg("num_ranges"), py::arg("flags"),
        py::arg("workspace"), py::arg("min_tiles"));
  m.def("set_library_error", &set_library_error);
}
