// rq_host.hpp -- C++ host layer above the librq C ABI, mirroring the Rust
// interface of runtimed's quantized linear path so that callers (and tests)
// read as they do against the reference:
//
//   GgufFile            crates/runtimed-gguf/src/header.rs:109-219
//   QMatMul             the q_map value, candle QMatMul::QTensor (load_gguf.rs:28-38)
//   Weights             crates/runtimed-model/src/weights/store.rs:12-166,
//                       linear_layer.rs:45-105, load_gguf.rs:40-120
//   Fp8Weight           crates/runtimed-model/src/weights/fp8_weight.rs:9-97
//   MarlinWeight        crates/runtimed-model/src/ops/marlin_gemv.rs:11-202
//   SubstratePort /
//   HipSubstrate        crates/runtimed-model/src/substrate/port.rs:14-77 (fp8_gemm,
//                       marlin_gemv)
//   ModelError/GgufError crates/runtimed-model/src/error.rs:5-27,
//                       crates/runtimed-gguf/src/error.rs:3-37
//
// Errors are thrown as exceptions carrying the reference's error kind.  Device
// memory is HIP memory on one ordinal; every call runs on the stream given at
// construction (default: the legacy stream).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rq.h"

namespace runtimed {

enum class DType { F32, F16, BF16, F8E4M3, U8, U32 };
size_t dtype_size(DType t);
int dtype_rq(DType t);  // rq_ftype, or -1

// GgufError (crates/runtimed-gguf/src/error.rs:3-37)
struct GgufError : std::runtime_error {
  enum Kind { Io, BadMagic, Version, Truncated, MetaType, Range, Overflow, Unsupported };
  Kind kind;
  GgufError(Kind k, const std::string &msg) : std::runtime_error(msg), kind(k) {}
  bool is_missing() const { return kind == Io; }
};

// ModelError (crates/runtimed-model/src/error.rs:5-27).  Candle is the
// reference's tensor-error variant ("tensor: ..."); this mirror raises it for
// a 2-D Q2_K or Q3_K tensor, which the reference hands to candle's QMatMul
// (load_gguf.rs:11-26) but librq has no decoder for: there is no candle here
// to hold it (the Rust binding keeps such tensors on candle).  Q4_1 and Q5_1
// never get that far: tensor_bytes has no geometry for them and fails with
// GgufError::Unsupported, here as in the reference (header.rs:191-194).
struct ModelError : std::runtime_error {
  enum Kind { Arch, Config, MissingWeight, Shape, Gguf, Candle };
  Kind kind;
  std::string name;
  std::vector<size_t> expected, got;
  ModelError(Kind k, const std::string &msg) : std::runtime_error(msg), kind(k) {}
  static ModelError shape(const std::string &name, std::vector<size_t> expected,
                          std::vector<size_t> got);
};

// A dense device tensor (row-major).  A tensor with no storage ("meta") only
// carries dims and dtype.
class Tensor {
 public:
  Tensor() = default;
  static Tensor zeros(std::vector<size_t> dims, DType t, int device);
  static Tensor from_host(const void *src, std::vector<size_t> dims, DType t, int device);
  static Tensor meta(std::vector<size_t> dims, DType t);
  std::vector<uint8_t> to_host() const;
  template <class T>
  std::vector<T> to_vec() const {
    auto b = to_host();
    return std::vector<T>(reinterpret_cast<const T *>(b.data()),
                          reinterpret_cast<const T *>(b.data() + b.size()));
  }
  const std::vector<size_t> &dims() const { return dims_; }
  size_t dim(size_t i) const { return dims_.at(i); }
  size_t elem_count() const;
  DType dtype() const { return dtype_; }
  int device() const { return device_; }
  void *data() const { return ptr_.get(); }
  bool has_storage() const { return ptr_ != nullptr; }
  // Same storage, other dims (same element count).
  Tensor reshaped(std::vector<size_t> dims) const;

 private:
  std::shared_ptr<void> ptr_;
  std::vector<size_t> dims_;
  DType dtype_ = DType::F32;
  int device_ = -1;
};

// MetaValue / TensorInfo / GgufFile (header.rs:14-39, 109-219), GGUF v3.
struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;  // [fast, slow]
  uint32_t dtype;              // GgmlDtype id
  uint64_t offset;             // absolute file offset
  size_t n_elements;
};

class GgufFile {
 public:
  static GgufFile open(const std::string &path);
  static GgufFile parse(std::vector<uint8_t> bytes);
  const TensorInfo *tensor(const std::string &name) const;
  // Bounds-checked raw bytes (header.rs:191-205).
  const uint8_t *tensor_bytes(const TensorInfo &info, size_t *len) const;
  std::vector<TensorInfo> tensors;
  std::map<std::string, std::string> meta_str;  // string-valued metadata
  uint64_t alignment = 32;

 private:
  static GgufFile parse_view(std::shared_ptr<const uint8_t> data, size_t size);
  std::shared_ptr<const uint8_t> data_;  // the mapped file (or parsed buffer)
  size_t size_ = 0;
};

// The quantized q_map value: a librq weight handle behind shared ownership
// (Arc<QMatMul> in store.rs:18).
class QMatMul {
 public:
  QMatMul(int qtype, const void *blocks, size_t nbytes, size_t n, size_t k, int device);
  Tensor forward(const Tensor &x, void *stream = nullptr) const;  // y = x W^T
  // y = x W^T + bias, linear_bias's add in the same launch (bias [n], F32 /
  // F16 / BF16, cast to y's dtype before the add).
  Tensor forward_bias(const Tensor &x, const Tensor &bias, void *stream = nullptr) const;
  Tensor dequantize(void *stream = nullptr) const;                // [n, k] f32
  // Rows ids of the dequantized matrix, [ids.size(), k] f32 (QMatMul::embedding).
  Tensor embedding(const std::vector<uint32_t> &ids, void *stream = nullptr) const;
  size_t storage_size_in_bytes() const;
  size_t n() const { return n_; }
  size_t k() const { return k_; }
  int device() const { return device_; }
  int qtype() const { return qtype_; }

 private:
  std::shared_ptr<rq_weight> w_;
  size_t n_, k_;
  int device_, qtype_;
};

// MarlinWeight (marlin_gemv.rs:11-63): packed U32 [ceil(in_dim/32), out_dim, 4],
// scales [out_dim] or [out_dim, 1] (F32 here).
class MarlinWeight {
 public:
  static MarlinWeight create(Tensor packed, Tensor scales, size_t in_dim, size_t out_dim);
  size_t resident_bytes() const;
  Tensor dequantize(void *stream = nullptr) const;  // [out_dim, in_dim] f32
  const Tensor &packed() const { return packed_; }
  const Tensor &scales() const { return scales_; }
  size_t in_dim() const { return in_dim_; }
  size_t out_dim() const { return out_dim_; }

 private:
  Tensor packed_, scales_;
  size_t in_dim_ = 0, out_dim_ = 0;
};

// repack_marlin_tiles (marlin_gemv.rs:66-97), run on the weight's device.
MarlinWeight repack_marlin_tiles(const Tensor &weight, const Tensor &scales, void *stream = nullptr);

// SubstratePort (port.rs:14-77): the FP8 and Marlin entries.
class SubstratePort {
 public:
  virtual ~SubstratePort() = default;
  virtual Tensor fp8_gemm(const Tensor &x, const Tensor &w, const Tensor *scale) const = 0;
  // marlin_gemv (marlin_gemv.rs:119-202): x @ (w * scale)^T in x's dtype.
  virtual Tensor marlin_gemv(const Tensor &x, const MarlinWeight &w) const = 0;
};

// librq behind the port: x is encoded with the reference's unscaled e4m3
// encoder (fp8_gemm.rs:94-101) unless per_token is set; output F16 when x is
// F16 or F8E4M3, else F32 (fp8_gemm.rs:106).
class HipSubstrate : public SubstratePort {
 public:
  explicit HipSubstrate(bool per_token = false, void *stream = nullptr)
      : per_token_(per_token), stream_(stream) {}
  Tensor fp8_gemm(const Tensor &x, const Tensor &w, const Tensor *scale) const override;
  Tensor marlin_gemv(const Tensor &x, const MarlinWeight &w) const override;

 private:
  bool per_token_;
  void *stream_;
};

// Fp8Weight (fp8_weight.rs:9-97).
class Fp8Weight {
 public:
  static Fp8Weight create(Tensor weight, Tensor scale, size_t in_dim, size_t out_dim);
  size_t in_dim() const { return in_dim_; }
  size_t out_dim() const { return out_dim_; }
  size_t resident_bytes() const;
  Tensor forward(const Tensor &x, const SubstratePort &port) const;
  const Tensor &weight() const { return weight_; }
  const Tensor &scale() const { return scale_; }

 private:
  Tensor weight_, scale_;
  size_t in_dim_ = 0, out_dim_ = 0;
};

// Weights (store.rs:12-19): dense map + quantized q_map.
class Weights {
 public:
  static Weights from_parts(int device, std::unordered_map<std::string, Tensor> map);
  static Weights from_quantized(int device, std::unordered_map<std::string, Tensor> map,
                                std::unordered_map<std::string, std::shared_ptr<QMatMul>> q_map);
  // load_gguf.rs:40-120: 2-D tensors in the block formats the reference maps
  // to candle (load_gguf.rs:11-26) become QMatMul handles (raw block bytes
  // uploaded as they are), or raise ModelError::Candle for Q2_K / Q3_K,
  // which librq does not decode; every other tensor goes the reference's
  // tensor_f32 way: F32 / F16 / BF16 uploaded as their dtype, block formats
  // decoded to F32 (GgufError::Unsupported where dequant_tensor has no
  // decoder, dequant.rs:143).  A missing output.weight aliases
  // token_embd.weight.
  static Weights load(const GgufFile &file, int device);

  Tensor linear(const Tensor &x, const std::string &name) const;        // linear_layer.rs:45-66
  // linear_layer.rs:107-118: linear, plus the tensor named *bias (if not
  // null) cast to y's dtype and broadcast-added; fused for quantized weights.
  Tensor linear_bias(const Tensor &x, const std::string &name, const std::string *bias) const;
  Tensor linear_dense(const Tensor &x, const std::string &name) const;  // linear_layer.rs:68-105
  Tensor get(const std::string &name) const;                            // store.rs:78-101
  // embed_layer.rs:16-57: rows ids as f32 [1, ids.size(), hidden].
  Tensor embed(const std::string &name, const std::vector<uint32_t> &ids) const;
  // embed_layer.rs:59-84: the same rows as [ids.size(), hidden].
  Tensor candidate_weights(const std::string &name, const std::vector<uint32_t> &ids) const;
  const Tensor &get_raw(const std::string &name) const;                 // store.rs:103-107
  // linear_layer.rs:17-22: registers packed and scales under the name's stem.
  void insert_marlin(const std::string &name, const MarlinWeight &mw);
  std::shared_ptr<QMatMul> q_matmul(const std::string &name) const;
  size_t resident_bytes() const;                                         // store.rs:57-76
  bool contains_key(const std::string &name) const;
  int device() const { return device_; }
  void set_substrate(std::shared_ptr<SubstratePort> s) { substrate_ = std::move(s); }

 private:
  // linear_layer.rs:24-42: the packed / scales pair under any of the
  // reference's key spellings, or null.
  bool find_marlin(const std::string &name, const Tensor **packed, const Tensor **scales) const;
  int device_ = 0;
  std::unordered_map<std::string, Tensor> map_;
  std::unordered_map<std::string, std::shared_ptr<QMatMul>> q_map_;
  std::shared_ptr<SubstratePort> substrate_ = std::make_shared<HipSubstrate>();
};

}  // namespace runtimed
