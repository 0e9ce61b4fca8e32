// rq_host.cpp -- the C++ host layer of rq_host.hpp over the librq C ABI.
#include "rq_host.hpp"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <fstream>
#include <iterator>
#include <unordered_set>

namespace runtimed {
namespace {

void hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) throw ModelError(ModelError::Config, std::string(what) + ": " + hipGetErrorString(e));
}

void rq_ok(int rc, const std::string &name, std::vector<size_t> expected = {},
           std::vector<size_t> got = {}) {
  if (rc == RQ_OK) return;
  const std::string msg = rq_last_error();
  if (rc == RQ_E_SHAPE) throw ModelError::shape(name, std::move(expected), std::move(got));
  throw ModelError(ModelError::Config, name + ": " + msg);
}

std::vector<size_t> leading(const std::vector<size_t> &d) {
  return std::vector<size_t>(d.begin(), d.end() - (d.empty() ? 0 : 1));
}

size_t product(const std::vector<size_t> &d) {
  size_t p = 1;
  for (size_t v : d) p *= v;
  return p;
}

// A dense F32 / F16 / BF16 tensor as F32 on its device (the to_dtype(F32) of
// fp8_gemm.rs and fp8_weight.rs:87-91).  16-bit values widen exactly: a
// zero F32 tensor plus the values through rq_bias_add (0 + b is b).
Tensor as_f32(const Tensor &t, const char *what) {
  if (t.dtype() == DType::F32) return t;
  const int bt = dtype_rq(t.dtype());
  if (bt != RQ_F16 && bt != RQ_BF16)
    throw ModelError(ModelError::Config, std::string(what) + ": dtype cannot be read as F32");
  Tensor out = Tensor::zeros(t.dims(), DType::F32, t.device());
  if (t.elem_count()) {
    hip_ok(hipSetDevice(t.device()), "hipSetDevice");
    rq_ok(rq_bias_add(out.data(), RQ_F32, 1, (int64_t)t.elem_count(), t.data(), bt, nullptr), what);
  }
  return out;
}

// GgmlDtype::block (dtype.rs:49-64)
bool block_geometry(uint32_t t, size_t *elems, size_t *bytes) {
  switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;
    case 1: case 30: *elems = 1; *bytes = 2; return true;
    case 2: *elems = 32; *bytes = 18; return true;
    case 6: *elems = 32; *bytes = 22; return true;
    case 8: *elems = 32; *bytes = 34; return true;
    case 10: *elems = 256; *bytes = 84; return true;
    case 11: *elems = 256; *bytes = 110; return true;
    case 12: *elems = 256; *bytes = 144; return true;
    case 13: *elems = 256; *bytes = 176; return true;
    case 14: *elems = 256; *bytes = 210; return true;
    default: return false;
  }
}

bool librq_decodes(uint32_t t) { return t == 2 || t == 6 || t == 8 || t == 12 || t == 13 || t == 14; }

// to_candle_quantized_dtype (load_gguf.rs:11-26): the block formats whose
// 2-D tensors the reference loads as candle QMatMul (Q4_1 and Q5_1 among
// them, though tensor_bytes rejects those first for want of a geometry).
bool candle_quantized(uint32_t t) { return (t >= 2 && t <= 3) || (t >= 6 && t <= 8) || (t >= 10 && t <= 14); }

const char *format_name(uint32_t t) {
  switch (t) {
    case 3: return "Q4_1";
    case 7: return "Q5_1";
    case 9: return "Q8_1";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 15: return "Q8_K";
    default: return "block format";
  }
}

// Cursor over the mapped bytes (header.rs:41-107).
struct Cursor {
  const uint8_t *data;
  size_t size;
  size_t pos = 0;
  const uint8_t *take(size_t n) {
    if (n > size - pos || pos > size) throw GgufError(GgufError::Truncated, "truncated file at offset " + std::to_string(pos));
    const uint8_t *p = data + pos;
    pos += n;
    return p;
  }
  template <class T>
  T get() {
    T v;
    std::memcpy(&v, take(sizeof(T)), sizeof(T));
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    const uint8_t *p = take(len);
    return std::string(reinterpret_cast<const char *>(p), len);
  }
  // Skips (or, for strings and u32, returns) one metadata value of type `ty`.
  void value(uint32_t ty, std::string *s, uint64_t *u) {
    switch (ty) {
      case 0: case 1: case 7: take(1); break;
      case 2: case 3: take(2); break;
      case 4: *u = get<uint32_t>(); break;
      case 5: case 6: take(4); break;
      case 8: *s = str(); break;
      case 9: {
        const uint32_t et = get<uint32_t>();
        const uint64_t n = get<uint64_t>();
        std::string ds;
        uint64_t du;
        for (uint64_t i = 0; i < n; ++i) value(et, &ds, &du);
        break;
      }
      case 10: case 11: case 12: take(8); break;
      default: throw GgufError(GgufError::MetaType, "unknown metadata type id: " + std::to_string(ty));
    }
  }
};

}  // namespace

size_t dtype_size(DType t) {
  switch (t) {
    case DType::F32: case DType::U32: return 4;
    case DType::F16: case DType::BF16: return 2;
    default: return 1;
  }
}

int dtype_rq(DType t) {
  switch (t) {
    case DType::F32: return RQ_F32;
    case DType::F16: return RQ_F16;
    case DType::BF16: return RQ_BF16;
    case DType::F8E4M3: case DType::U8: return RQ_F8E4M3;
    default: return -1;
  }
}

ModelError ModelError::shape(const std::string &name, std::vector<size_t> expected,
                             std::vector<size_t> got) {
  ModelError e(Shape, "shape mismatch on " + name);
  e.name = name;
  e.expected = std::move(expected);
  e.got = std::move(got);
  return e;
}

// ------------------------------------------------------------------ Tensor --

size_t Tensor::elem_count() const { return product(dims_); }

Tensor Tensor::reshaped(std::vector<size_t> dims) const {
  if (product(dims) != elem_count()) throw ModelError::shape("reshape", dims, dims_);
  Tensor r = *this;
  r.dims_ = std::move(dims);
  return r;
}

Tensor Tensor::zeros(std::vector<size_t> dims, DType t, int device) {
  Tensor r;
  r.dims_ = std::move(dims);
  r.dtype_ = t;
  r.device_ = device;
  const size_t bytes = r.elem_count() * dtype_size(t);
  hip_ok(hipSetDevice(device), "hipSetDevice");
  void *p = nullptr;
  hip_ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
  r.ptr_ = std::shared_ptr<void>(p, [device](void *q) {
    int cur = 0;
    if (hipGetDevice(&cur) == hipSuccess && cur != device) (void)hipSetDevice(device);
    (void)hipFree(q);
    if (cur != device) (void)hipSetDevice(cur);
  });
  if (bytes) hip_ok(hipMemset(p, 0, bytes), "hipMemset");
  return r;
}

Tensor Tensor::from_host(const void *src, std::vector<size_t> dims, DType t, int device) {
  Tensor r = zeros(std::move(dims), t, device);
  const size_t bytes = r.elem_count() * dtype_size(t);
  if (bytes) hip_ok(hipMemcpy(r.data(), src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return r;
}

Tensor Tensor::meta(std::vector<size_t> dims, DType t) {
  Tensor r;
  r.dims_ = std::move(dims);
  r.dtype_ = t;
  return r;
}

std::vector<uint8_t> Tensor::to_host() const {
  std::vector<uint8_t> out(elem_count() * dtype_size(dtype_));
  if (!has_storage()) throw ModelError(ModelError::Config, "tensor has no storage");
  hip_ok(hipSetDevice(device_), "hipSetDevice");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  if (!out.empty()) hip_ok(hipMemcpy(out.data(), data(), out.size(), hipMemcpyDeviceToHost), "hipMemcpy");
  return out;
}

// ---------------------------------------------------------------- GgufFile --

// The file is memory-mapped read-only (as header.rs maps it) with its pages
// populated up front, so tensor bytes go to the upload without a copy.
GgufFile GgufFile::open(const std::string &path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) throw GgufError(GgufError::Io, "io: cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    throw GgufError(GgufError::Io, "io: cannot stat " + path);
  }
  const size_t size = (size_t)st.st_size;
  if (size == 0) {
    ::close(fd);
    return parse(std::vector<uint8_t>());
  }
  void *p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE | MAP_POPULATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) throw GgufError(GgufError::Io, "io: cannot map " + path);
  std::shared_ptr<const uint8_t> data(static_cast<const uint8_t *>(p), [size](const uint8_t *q) {
    munmap(const_cast<uint8_t *>(q), size);
  });
  return parse_view(std::move(data), size);
}

GgufFile GgufFile::parse(std::vector<uint8_t> bytes) {
  auto owned = std::make_shared<std::vector<uint8_t>>(std::move(bytes));
  std::shared_ptr<const uint8_t> data(owned, owned->data());
  return parse_view(std::move(data), owned->size());
}

GgufFile GgufFile::parse_view(std::shared_ptr<const uint8_t> data, size_t size) {
  GgufFile g;
  g.data_ = std::move(data);
  g.size_ = size;
  Cursor cur{g.data_.get(), g.size_};
  if (std::memcmp(cur.take(4), "GGUF", 4) != 0) throw GgufError(GgufError::BadMagic, "bad magic: not a GGUF file");
  const uint32_t version = cur.get<uint32_t>();
  if (version != 3) throw GgufError(GgufError::Version, "unsupported GGUF version: " + std::to_string(version) + " (want 3)");
  const uint64_t n_tensors = cur.get<uint64_t>();
  const uint64_t n_meta = cur.get<uint64_t>();
  uint64_t align = 32;
  for (uint64_t i = 0; i < n_meta; ++i) {
    const std::string key = cur.str();
    const uint32_t ty = cur.get<uint32_t>();
    std::string s;
    uint64_t u = 0;
    cur.value(ty, &s, &u);
    if (ty == 8) g.meta_str[key] = s;
    if (key == "general.alignment" && ty == 4) align = u;  // header.rs:162-166
  }
  if (align == 0) align = 1;
  struct Raw { std::string name; std::vector<uint64_t> dims; uint32_t dtype; uint64_t off; };
  std::vector<Raw> raws;
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Raw r;
    r.name = cur.str();
    const uint32_t nd = cur.get<uint32_t>();
    if (nd > 8) throw GgufError(GgufError::Truncated, "truncated file at offset " + std::to_string(cur.pos));
    for (uint32_t d = 0; d < nd; ++d) r.dims.push_back(cur.get<uint64_t>());
    r.dtype = cur.get<uint32_t>();
    r.off = cur.get<uint64_t>();
    raws.push_back(std::move(r));
  }
  const uint64_t data_start = (cur.pos + align - 1) / align * align;
  g.alignment = align;
  for (auto &r : raws) {
    size_t n = 1;
    for (uint64_t d : r.dims) {
      if (d != 0 && n > SIZE_MAX / d) throw GgufError(GgufError::Overflow, "tensor '" + r.name + "': element count overflows");
      n *= d;
    }
    const uint64_t off = data_start + r.off;
    if (off < data_start || off > g.size_) throw GgufError(GgufError::Range, "tensor '" + r.name + "': byte range out of bounds");
    g.tensors.push_back(TensorInfo{r.name, r.dims, r.dtype, off, n});
  }
  return g;
}

const TensorInfo *GgufFile::tensor(const std::string &name) const {
  for (const auto &t : tensors)
    if (t.name == name) return &t;
  return nullptr;
}

const uint8_t *GgufFile::tensor_bytes(const TensorInfo &info, size_t *len) const {
  size_t elems, bb;
  if (!block_geometry(info.dtype, &elems, &bb)) throw GgufError(GgufError::Unsupported, "decode of dtype " + std::to_string(info.dtype) + " not implemented");
  const size_t blocks = (info.n_elements + elems - 1) / elems;
  if (blocks > SIZE_MAX / bb) throw GgufError(GgufError::Overflow, "tensor '" + info.name + "': element count overflows");
  const size_t n = blocks * bb;
  if (info.offset > size_ || n > size_ - info.offset) throw GgufError(GgufError::Range, "tensor '" + info.name + "': byte range out of bounds");
  *len = n;
  return data_.get() + info.offset;
}

// ----------------------------------------------------------------- QMatMul --

QMatMul::QMatMul(int qtype, const void *blocks, size_t nbytes, size_t n, size_t k, int device)
    : n_(n), k_(k), device_(device), qtype_(qtype) {
  rq_weight *h = nullptr;
  rq_ok(rq_weight_create(qtype, blocks, nbytes, (int64_t)n, (int64_t)k, device, &h), "rq_weight_create",
        {n, k}, {nbytes});
  w_ = std::shared_ptr<rq_weight>(h, rq_weight_destroy);
}

Tensor QMatMul::forward(const Tensor &x, void *stream) const {
  if (x.dims().empty() || x.dims().back() != k_) throw ModelError::shape("qmatmul", {k_}, x.dims());
  const int xt = dtype_rq(x.dtype());
  if (xt != RQ_F32 && xt != RQ_F16 && xt != RQ_BF16) throw ModelError(ModelError::Config, "activation dtype not supported");
  auto dims = leading(x.dims());
  dims.push_back(n_);
  Tensor y = Tensor::zeros(dims, x.dtype(), device_);
  rq_ok(rq_linear(w_.get(), x.data(), xt, (int64_t)(x.elem_count() / k_), (int64_t)x.dims().back(), y.data(), xt,
                  stream),
        "linear", {k_}, x.dims());
  return y;
}

Tensor QMatMul::forward_bias(const Tensor &x, const Tensor &bias, void *stream) const {
  if (x.dims().empty() || x.dims().back() != k_) throw ModelError::shape("qmatmul", {k_}, x.dims());
  if (bias.elem_count() != n_) throw ModelError::shape("bias", {n_}, bias.dims());
  const int xt = dtype_rq(x.dtype()), bt = dtype_rq(bias.dtype());
  if (xt != RQ_F32 && xt != RQ_F16 && xt != RQ_BF16) throw ModelError(ModelError::Config, "activation dtype not supported");
  if (bt != RQ_F32 && bt != RQ_F16 && bt != RQ_BF16) throw ModelError(ModelError::Config, "bias dtype not supported");
  if (bias.device() != device_) throw ModelError(ModelError::Config, "bias on another device");
  auto dims = leading(x.dims());
  dims.push_back(n_);
  Tensor y = Tensor::zeros(dims, x.dtype(), device_);
  rq_ok(rq_linear_bias(w_.get(), x.data(), xt, (int64_t)(x.elem_count() / k_), (int64_t)x.dims().back(),
                       bias.data(), bt, y.data(), xt, stream),
        "linear_bias", {k_}, x.dims());
  return y;
}

Tensor QMatMul::dequantize(void *stream) const {
  Tensor out = Tensor::zeros({n_, k_}, DType::F32, device_);
  rq_ok(rq_dequant_f32(w_.get(), static_cast<float *>(out.data()), stream), "dequantize");
  return out;
}

Tensor QMatMul::embedding(const std::vector<uint32_t> &ids, void *stream) const {
  Tensor out = Tensor::zeros({ids.size(), k_}, DType::F32, device_);
  if (ids.empty()) return out;
  const int rc = rq_embedding(w_.get(), ids.data(), (int64_t)ids.size(), static_cast<float *>(out.data()), stream);
  if (rc == RQ_E_ARG) throw ModelError(ModelError::Shape, std::string("embedding: ") + rq_last_error());
  rq_ok(rc, "embedding");
  return out;
}

size_t QMatMul::storage_size_in_bytes() const {
  rq_weight_desc d;
  rq_ok(rq_weight_info(w_.get(), &d), "rq_weight_info");
  return (size_t)d.device_bytes;
}

// ------------------------------------------------------------ HipSubstrate --

Tensor HipSubstrate::fp8_gemm(const Tensor &x, const Tensor &w, const Tensor *scale) const {
  if (w.dims().size() != 2) throw ModelError::shape("fp8_gemm", {0, 0}, w.dims());
  const size_t n = w.dim(0), k = w.dim(1);
  if (x.dims().empty() || x.dims().back() != k) throw ModelError::shape("fp8_gemm", {k}, x.dims());
  const size_t m = x.elem_count() / k;
  // fp8_gemm.rs:106: F16 out for F16/F8 activations, else F32.
  const DType out_dt = (x.dtype() == DType::F16 || x.dtype() == DType::F8E4M3) ? DType::F16 : DType::F32;
  auto dims = leading(x.dims());
  dims.push_back(n);
  Tensor y = Tensor::zeros(dims, out_dt, w.device());
  Tensor per_row, s32;
  const float *sp = nullptr;
  // The scale is read as F32 whatever its dtype (fp8_gemm.rs converts it
  // with to_dtype(F32)).
  if (scale && (scale->elem_count() == n || scale->elem_count() == 1)) s32 = as_f32(*scale, "fp8_scale");
  if (scale && scale->elem_count() == n) {
    sp = static_cast<const float *>(s32.data());
  } else if (scale && scale->elem_count() == 1) {  // per-tensor scale (fp8_gemm.rs:128-132)
    const float s = s32.to_vec<float>().at(0);
    std::vector<float> v(n, s);
    per_row = Tensor::from_host(v.data(), {n}, DType::F32, w.device());
    sp = static_cast<const float *>(per_row.data());
  } else if (scale) {
    throw ModelError::shape("fp8_scale", {n}, scale->dims());
  }
  rq_ok(rq_fp8_gemm(x.data(), dtype_rq(x.dtype()), (int64_t)m, static_cast<const uint8_t *>(w.data()), sp,
                    (int64_t)n, (int64_t)k, y.data(), dtype_rq(out_dt),
                    per_token_ ? RQ_FP8_PER_TOKEN : RQ_FP8_UNSCALED, stream_),
        "fp8_gemm", {k}, x.dims());
  return y;
}

Tensor HipSubstrate::marlin_gemv(const Tensor &x, const MarlinWeight &w) const {
  const size_t in_dim = x.dims().empty() ? 0 : x.dims().back();
  if (in_dim != w.in_dim()) throw ModelError::shape("marlin_gemv", {w.in_dim()}, x.dims());
  const size_t rows = in_dim ? x.elem_count() / in_dim : 0;
  auto dims = leading(x.dims());
  dims.push_back(w.out_dim());
  Tensor y = Tensor::zeros(dims, x.dtype(), w.packed().device());
  if (rows == 0 || w.out_dim() == 0) return y;
  const int xt = dtype_rq(x.dtype());
  if (xt != RQ_F32 && xt != RQ_F16 && xt != RQ_BF16) throw ModelError(ModelError::Config, "marlin: activation dtype");
  rq_ok(rq_marlin_linear(static_cast<const uint32_t *>(w.packed().data()), static_cast<const float *>(w.scales().data()),
                         (int64_t)w.out_dim(), (int64_t)in_dim, x.data(), xt, (int64_t)rows, y.data(), xt, stream_),
        "marlin_gemv", {w.in_dim()}, x.dims());
  return y;
}

// ------------------------------------------------------------ MarlinWeight --

MarlinWeight MarlinWeight::create(Tensor packed, Tensor scales, size_t in_dim, size_t out_dim) {
  if (packed.dtype() != DType::U32) throw ModelError(ModelError::Config, "marlin packed must be U32");
  if (scales.dims() != std::vector<size_t>{out_dim} && scales.dims() != std::vector<size_t>{out_dim, 1})
    throw ModelError::shape("marlin_scales", {out_dim}, scales.dims());
  if (scales.dtype() != DType::F32) throw ModelError(ModelError::Config, "marlin scales must be F32");
  if (packed.device() != scales.device())
    throw ModelError(ModelError::Config, "packed and scales must be on the same device");
  const size_t k_chunks = (in_dim + 31) / 32;
  if (packed.elem_count() < k_chunks * out_dim * 4)
    throw ModelError::shape("marlin_packed", {k_chunks, out_dim, 4}, packed.dims());
  MarlinWeight mw;
  mw.packed_ = std::move(packed);
  mw.scales_ = std::move(scales);
  mw.in_dim_ = in_dim;
  mw.out_dim_ = out_dim;
  return mw;
}

size_t MarlinWeight::resident_bytes() const {
  return packed_.elem_count() * dtype_size(packed_.dtype()) + scales_.elem_count() * dtype_size(scales_.dtype());
}

Tensor MarlinWeight::dequantize(void *stream) const {
  Tensor out = Tensor::zeros({out_dim_, in_dim_}, DType::F32, packed_.device());
  if (out_dim_ == 0 || in_dim_ == 0) return out;
  rq_ok(rq_marlin_dequant(static_cast<const uint32_t *>(packed_.data()), static_cast<const float *>(scales_.data()),
                          (int64_t)out_dim_, (int64_t)in_dim_, static_cast<float *>(out.data()), stream),
        "marlin_dequant");
  return out;
}

MarlinWeight repack_marlin_tiles(const Tensor &weight, const Tensor &scales, void *stream) {
  if (weight.dims().size() != 2) throw ModelError(ModelError::Config, "weight must be 2D");
  const size_t out_dim = weight.dim(0), in_dim = weight.dim(1);
  if (scales.elem_count() != out_dim) throw ModelError::shape("scales", {out_dim}, {scales.elem_count()});
  if (scales.dtype() != DType::F32) throw ModelError(ModelError::Config, "marlin scales must be F32");
  const int wt = dtype_rq(weight.dtype());
  if (wt != RQ_F32 && wt != RQ_F16 && wt != RQ_BF16) throw ModelError(ModelError::Config, "marlin: weight dtype");
  const size_t k_chunks = (in_dim + 31) / 32;
  Tensor packed = Tensor::zeros({k_chunks, out_dim, 4}, DType::U32, weight.device());
  if (out_dim && in_dim)
    rq_ok(rq_marlin_repack(weight.data(), wt, static_cast<const float *>(scales.data()), (int64_t)out_dim,
                           (int64_t)in_dim, static_cast<uint32_t *>(packed.data()), stream),
          "repack_marlin_tiles");
  return MarlinWeight::create(std::move(packed), scales, in_dim, out_dim);
}

// --------------------------------------------------------------- Fp8Weight --

Fp8Weight Fp8Weight::create(Tensor weight, Tensor scale, size_t in_dim, size_t out_dim) {
  if (weight.dims() != std::vector<size_t>{out_dim, in_dim})
    throw ModelError::shape("fp8_weight", {out_dim, in_dim}, weight.dims());
  if (scale.dims() != std::vector<size_t>{out_dim} && scale.dims() != std::vector<size_t>{out_dim, 1})
    throw ModelError::shape("fp8_scale", {out_dim}, scale.dims());
  const int st = dtype_rq(scale.dtype());
  if (st != RQ_F32 && st != RQ_F16 && st != RQ_BF16)
    throw ModelError(ModelError::Config, "fp8_scale: dtype cannot be read as F32");
  // Kept in its own dtype (resident_bytes counts it so, fp8_weight.rs:63-66);
  // fp8_gemm reads it as F32.
  Fp8Weight f;
  f.weight_ = std::move(weight);
  f.scale_ = std::move(scale);
  f.in_dim_ = in_dim;
  f.out_dim_ = out_dim;
  return f;
}

size_t Fp8Weight::resident_bytes() const {
  return weight_.elem_count() * dtype_size(weight_.dtype()) + scale_.elem_count() * dtype_size(scale_.dtype());
}

Tensor Fp8Weight::forward(const Tensor &x, const SubstratePort &port) const {
  return port.fp8_gemm(x, weight_, &scale_);
}

// ----------------------------------------------------------------- Weights --

Weights Weights::from_parts(int device, std::unordered_map<std::string, Tensor> map) {
  Weights w;
  w.device_ = device;
  w.map_ = std::move(map);
  return w;
}

Weights Weights::from_quantized(int device, std::unordered_map<std::string, Tensor> map,
                                std::unordered_map<std::string, std::shared_ptr<QMatMul>> q_map) {
  Weights w = from_parts(device, std::move(map));
  w.q_map_ = std::move(q_map);
  return w;
}

Weights Weights::load(const GgufFile &file, int device) {
  Weights w;
  w.device_ = device;
  const bool untied = file.tensor("output.weight") != nullptr;
  for (const auto &info : file.tensors) {
    size_t len = 0;
    const uint8_t *raw = file.tensor_bytes(info, &len);
    if (info.dims.size() == 2 && candle_quantized(info.dtype)) {
      if (!librq_decodes(info.dtype))
        throw ModelError(ModelError::Candle, "tensor '" + info.name + "': " + format_name(info.dtype) + " (dtype " +
                                                 std::to_string(info.dtype) +
                                                 ") is a candle-only block format: librq has no decoder for it");
      auto q = std::make_shared<QMatMul>((int)info.dtype, raw, len, (size_t)info.dims[1], (size_t)info.dims[0], device);
      if (info.name == "token_embd.weight" && !untied) w.q_map_["output.weight"] = q;  // load_gguf.rs:89-97
      w.q_map_[info.name] = q;
      continue;
    }
    std::vector<size_t> dims(info.dims.rbegin(), info.dims.rend());
    Tensor dense;
    if (info.dtype == 0 || info.dtype == 1 || info.dtype == 30) {
      const DType t = info.dtype == 0 ? DType::F32 : info.dtype == 1 ? DType::F16 : DType::BF16;
      dense = Tensor::from_host(raw, dims, t, device);
    } else {
      // tensor_f32 (header.rs:207-211): dequant_tensor to f32, with its errors
      if (!librq_decodes(info.dtype))
        throw GgufError(GgufError::Unsupported, "tensor '" + info.name + "': " + format_name(info.dtype) +
                                                    " (dtype " + std::to_string(info.dtype) + ") does not decode");
      dense = QMatMul((int)info.dtype, raw, len, 1, info.n_elements, device).dequantize().reshaped(dims);
    }
    if (info.name == "token_embd.weight" && !untied) w.map_["output.weight"] = dense;
    w.map_[info.name] = dense;
  }
  return w;
}

const Tensor &Weights::get_raw(const std::string &name) const {
  auto it = map_.find(name);
  if (it == map_.end()) throw ModelError(ModelError::MissingWeight, "missing weight: " + name);
  return it->second;
}

std::shared_ptr<QMatMul> Weights::q_matmul(const std::string &name) const {
  auto it = q_map_.find(name);
  return it == q_map_.end() ? nullptr : it->second;
}

bool Weights::contains_key(const std::string &name) const {
  return map_.count(name) != 0 || q_map_.count(name) != 0;
}

size_t Weights::resident_bytes() const {
  size_t dense = 0;
  for (const auto &kv : map_) dense += kv.second.elem_count() * dtype_size(kv.second.dtype());
  std::unordered_set<const QMatMul *> seen;
  size_t quant = 0;
  for (const auto &kv : q_map_)
    if (seen.insert(kv.second.get()).second) quant += kv.second->storage_size_in_bytes();
  return dense + quant;
}

Tensor Weights::get(const std::string &name) const {
  auto it = map_.find(name);
  if (it != map_.end()) return as_f32(it->second, "get");  // store.rs:79-86: dense tensors read as F32
  auto q = q_map_.find(name);
  if (q != q_map_.end()) return q->second->dequantize();
  throw ModelError(ModelError::MissingWeight, "missing weight: " + name);
}

Tensor Weights::candidate_weights(const std::string &name, const std::vector<uint32_t> &ids) const {
  auto q = q_map_.find(name);
  if (q != q_map_.end()) return q->second->embedding(ids);
  const Tensor &w = get_raw(name);
  if (w.dims().size() != 2) throw ModelError::shape(name, {0, 0}, w.dims());
  if (w.dtype() != DType::F32)
    throw ModelError(ModelError::Config, "embedding rows: only f32 dense tables are served here: " + name);
  const size_t hidden = w.dim(1), rows = w.dim(0);
  Tensor out = Tensor::zeros({ids.size(), hidden}, DType::F32, w.device());
  for (size_t i = 0; i < ids.size(); ++i) {
    if (ids[i] >= rows)
      throw ModelError(ModelError::Shape, "embedding: id " + std::to_string(ids[i]) + " out of range for " +
                                              std::to_string(rows) + " rows of " + name);
    hip_ok(hipMemcpyAsync(static_cast<float *>(out.data()) + i * hidden,
                          static_cast<const float *>(w.data()) + (size_t)ids[i] * hidden, hidden * sizeof(float),
                          hipMemcpyDeviceToDevice, nullptr),
           "hipMemcpyAsync");
  }
  return out;
}

Tensor Weights::embed(const std::string &name, const std::vector<uint32_t> &ids) const {
  Tensor rows = candidate_weights(name, ids);
  return rows.reshaped({1, rows.dim(0), rows.dim(1)});
}

void Weights::insert_marlin(const std::string &name, const MarlinWeight &mw) {
  const std::string suffix = ".weight";
  const bool has = name.size() >= suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0;
  const std::string stem = has ? name.substr(0, name.size() - suffix.size()) : name;
  map_[name] = mw.packed();
  map_[stem + ".marlin_packed"] = mw.packed();
  map_[stem + ".marlin_scales"] = mw.scales();
}

bool Weights::find_marlin(const std::string &name, const Tensor **packed, const Tensor **scales) const {
  const std::string suffix = ".weight";
  const bool has = name.size() >= suffix.size() && name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0;
  const std::string stem = has ? name.substr(0, name.size() - suffix.size()) : name;
  auto get = [&](const std::string &key, bool want_u32) -> const Tensor * {
    auto it = map_.find(key);
    if (it == map_.end() || (want_u32 && it->second.dtype() != DType::U32)) return nullptr;
    return &it->second;
  };
  const Tensor *p = nullptr;
  for (const std::string &key : {name + ".marlin_packed", stem + ".marlin_packed", name + ".packed", stem + ".packed"})
    if (!p) p = get(key, false);
  if (!p) p = get(name, true);
  if (!p) p = get(stem, true);
  if (!p) return false;
  const Tensor *sc = nullptr;
  for (const std::string &key : {name + ".marlin_scales", stem + ".marlin_scales", name + ".scales", stem + ".scales",
                                 name + ".scale", stem + ".scale", name + ".weight.scale", stem + ".weight.scale"})
    if (!sc) sc = get(key, false);
  if (!sc) return false;
  *packed = p;
  *scales = sc;
  return true;
}

Tensor Weights::linear(const Tensor &x, const std::string &name) const {
  auto q = q_map_.find(name);
  if (q != q_map_.end()) return q->second->forward(x);
  const Tensor *packed = nullptr, *scales = nullptr;
  if (find_marlin(name, &packed, &scales)) {
    // linear_layer.rs:53-63: in_dim comes from x, checked against the
    // number of packed chunks.
    const size_t x_in = x.dims().empty() ? 0 : x.dims().back();
    const size_t out_dim = scales->elem_count();
    const size_t k_chunks = packed->dims().size() >= 2 ? packed->dim(0) : (x_in + 31) / 32;
    const size_t max_k = k_chunks * 32, min_k = k_chunks > 1 ? (k_chunks - 1) * 32 : 0;
    if (x_in > max_k || (k_chunks > 1 && x_in <= min_k)) throw ModelError::shape(name, {max_k}, x.dims());
    return substrate_->marlin_gemv(x, MarlinWeight::create(*packed, *scales, x_in, out_dim));
  }
  return linear_dense(x, name);
}

Tensor Weights::linear_bias(const Tensor &x, const std::string &name, const std::string *bias) const {
  if (!bias) return linear(x, name);
  const Tensor b = get(*bias);
  auto q = q_map_.find(name);
  if (q != q_map_.end()) return q->second->forward_bias(x, b);
  // Other paths: the linear, then the bias cast to y's dtype and added.
  Tensor y = linear(x, name);
  const size_t n = y.dims().empty() ? 0 : y.dims().back();
  if (b.elem_count() != n) throw ModelError::shape(*bias, {n}, b.dims());
  const int bt = dtype_rq(b.dtype()), yt = dtype_rq(y.dtype());
  if (bt != RQ_F32 && bt != RQ_F16 && bt != RQ_BF16) throw ModelError(ModelError::Config, "bias dtype not supported");
  hip_ok(hipSetDevice(y.device()), "hipSetDevice");
  rq_ok(rq_bias_add(y.data(), yt, (int64_t)(n ? y.elem_count() / n : 0), (int64_t)n, b.data(), bt, nullptr),
        "linear_bias");
  return y;
}

Tensor Weights::linear_dense(const Tensor &x, const std::string &name) const {
  const Tensor *packed = nullptr, *scales = nullptr;
  if (find_marlin(name, &packed, &scales)) {  // linear_layer.rs:69-74
    const size_t x_in = x.dims().empty() ? 0 : x.dims().back();
    return substrate_->marlin_gemv(x, MarlinWeight::create(*packed, *scales, x_in, scales->elem_count()));
  }
  const Tensor &w = get_raw(name);
  if (w.dtype() == DType::F8E4M3 || w.dtype() == DType::U8) {
    // scale lookup order of linear_layer.rs:79-85; absent = ones
    for (const char *suf : {".scale", "_scale", ".weight_scale_inv"}) {
      auto s = map_.find(name + suf);
      if (s != map_.end()) return substrate_->fp8_gemm(x, w, &s->second);
    }
    return substrate_->fp8_gemm(x, w, nullptr);
  }
  throw ModelError(ModelError::Config, "dense " + name + ": only quantized and F8E4M3 weights run on this path");
}

}  // namespace runtimed
