// test_host.cpp -- tests of the C++ host layer (runtimed_amd/host), written
// after the reference's own unit tests.  `--cpu` runs the tests that need no
// device (GGUF parsing, shape checks); `--gpu` runs the device tests, checked
// against the oracle (oracle/rq_oracle.h).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <string>
#include <vector>

#include "../../oracle/rq_oracle.h"
#include "../../runtimed_amd/host/rq_host.hpp"

using namespace runtimed;

static int g_fail = 0, g_run = 0;
#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      std::fprintf(stderr, "  check failed %s:%d: %s\n", __FILE__, __LINE__, #c); \
      throw std::runtime_error("check failed");                           \
    }                                                                     \
  } while (0)

static void run(const char *name, const std::function<void()> &f) {
  ++g_run;
  std::printf("%s ... ", name);
  std::fflush(stdout);
  try {
    f();
    std::printf("ok\n");
  } catch (const std::exception &e) {
    ++g_fail;
    std::printf("FAILED (%s)\n", e.what());
  }
  std::fflush(stdout);
}

template <class E, class F>
static E expect_throw(F f) {
  try {
    f();
  } catch (const E &e) {
    return e;
  }
  throw std::runtime_error("expected exception not thrown");
}

// ---- forged GGUF files (the pattern of tests/integration/arch_config.rs) ----
struct GgufWriter {
  std::vector<uint8_t> b;
  void u32(uint32_t v) { put(&v, 4); }
  void u64(uint64_t v) { put(&v, 8); }
  void put(const void *p, size_t n) { b.insert(b.end(), (const uint8_t *)p, (const uint8_t *)p + n); }
  void str(const std::string &s) { u64(s.size()); put(s.data(), s.size()); }
};

struct ForgedTensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t dtype;
  std::vector<uint8_t> data;
};

static std::vector<uint8_t> forge(const std::vector<ForgedTensor> &ts, uint32_t align = 32,
                                  uint32_t version = 3) {
  GgufWriter w;
  w.put("GGUF", 4);
  w.u32(version);
  w.u64(ts.size());
  w.u64(2);
  w.str("general.alignment");
  w.u32(4);
  w.u32(align);
  w.str("general.name");
  w.u32(8);
  w.str("forged");
  uint64_t off = 0;
  std::vector<uint64_t> offs;
  for (const auto &t : ts) {
    off = (off + align - 1) / align * align;
    offs.push_back(off);
    off += t.data.size();
  }
  for (size_t i = 0; i < ts.size(); ++i) {
    w.str(ts[i].name);
    w.u32((uint32_t)ts[i].dims.size());
    for (auto d : ts[i].dims) w.u64(d);
    w.u32(ts[i].dtype);
    w.u64(offs[i]);
  }
  while (w.b.size() % align) w.b.push_back(0);
  const size_t base = w.b.size();
  for (size_t i = 0; i < ts.size(); ++i) {
    w.b.resize(base + offs[i], 0);
    w.put(ts[i].data.data(), ts[i].data.size());
  }
  return w.b;
}

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {
  g_rng += 0x9E3779B97F4A7C15ull;
  uint64_t z = g_rng;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static uint16_t f16_of(float f) {  // finite positive normal range only
  _Float16 h = (_Float16)f;
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}
static std::vector<uint8_t> rand_blocks(uint32_t dtype, size_t nblocks) {
  size_t elems, bytes;
  rqo_block_geometry(dtype, &elems, &bytes);
  std::vector<uint8_t> b(nblocks * bytes);
  for (auto &v : b) v = (uint8_t)next_u64();
  for (size_t i = 0; i < nblocks; ++i) {
    uint8_t *blk = b.data() + i * bytes;
    const float u = 1e-4f + 1e-2f * (float)((next_u64() >> 11) * (1.0 / 9007199254740992.0));
    const uint16_t h = f16_of(u);
    if (dtype == 14) std::memcpy(blk + 208, &h, 2);   // Q6_K d
    else std::memcpy(blk, &h, 2);                     // Q8_0/Q4_K d
    if (dtype == 12) std::memcpy(blk + 2, &h, 2);     // Q4_K dmin
  }
  return b;
}
static std::vector<float> rand_normal(size_t n) {
  std::vector<float> v(n);
  for (auto &x : v) {
    const double u1 = ((next_u64() >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (next_u64() >> 11) * (1.0 / 9007199254740992.0);
    x = (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
  return v;
}
static double norm_err(const std::vector<float> &y, const std::vector<double> &r) {
  double mx = 0, md = 0;
  for (size_t i = 0; i < r.size(); ++i) {
    mx = std::fmax(mx, std::fabs(r[i]));
    md = std::fmax(md, std::fabs((double)y[i] - r[i]));
  }
  return mx > 0 ? md / mx : md;
}

// ----------------------------------------------------------------- CPU ------

static void cpu_tests() {
  run("open_missing_file_errors", [] {  // header.rs:229-233
    auto e = expect_throw<GgufError>([] { GgufFile::open("/nonexistent/runtimed-gguf-test.gguf"); });
    CHECK(e.is_missing());
  });
  run("open_non_gguf_rejects_bad_magic", [] {  // header.rs:235-242
    const std::string p = "/tmp/rq-host-bad-magic.gguf";
    { std::ofstream(p, std::ios::binary) << "not-a-gguf-file-payload"; }
    auto e = expect_throw<GgufError>([&] { GgufFile::open(p); });
    std::remove(p.c_str());
    CHECK(e.kind == GgufError::BadMagic);
  });
  run("rejects_version_2", [] {
    auto e = expect_throw<GgufError>([] { GgufFile::parse(forge({}, 32, 2)); });
    CHECK(e.kind == GgufError::Version);
  });
  run("forged_file_tensor_ranges", [] {
    auto q4 = rand_blocks(12, 4);
    std::vector<uint8_t> f32(256 * 4, 0);
    auto g = GgufFile::parse(forge({{"blk.0.ffn_up.weight", {256, 4}, 12, q4},
                                    {"output_norm.weight", {256}, 0, f32}}, 64));
    CHECK(g.alignment == 64);
    CHECK(g.meta_str.at("general.name") == "forged");
    const TensorInfo *t = g.tensor("blk.0.ffn_up.weight");
    CHECK(t && t->n_elements == 1024 && t->dtype == 12 && t->dims.size() == 2 && t->dims[1] == 4);
    size_t len = 0;
    const uint8_t *p = g.tensor_bytes(*t, &len);
    CHECK(len == 4 * 144 && std::memcmp(p, q4.data(), len) == 0);
    const TensorInfo *n = g.tensor("output_norm.weight");
    CHECK(n && n->offset % 64 == 0 && n->offset - t->offset == 576);
    CHECK(g.tensor("missing") == nullptr);
  });
  run("load_formats_without_a_librq_decoder", [] {  // load_gguf.rs:11-26, header.rs:191-211
    // Q2_K / Q3_K: the reference loads them into candle's QMatMul; librq has
    // no decoder, so the mirror raises its distinct ModelError::Candle
    for (uint32_t t : {10u, 11u}) {
      std::vector<uint8_t> data(2 * (t == 10 ? 84 : 110), 0x11);
      auto g = GgufFile::parse(forge({{"blk.0.ffn_up.weight", {256, 2}, t, data}}));
      auto e = expect_throw<ModelError>([&] { Weights::load(g, 0); });
      CHECK(e.kind == ModelError::Candle);
      CHECK(std::string(e.what()).find("candle-only") != std::string::npos);
    }
    // Q4_1 / Q5_1 (mapped to candle too) and Q8_1 (not mapped): tensor_bytes
    // has no geometry for them, GgufError::Unsupported as in the reference
    for (uint32_t t : {3u, 7u, 9u}) {
      std::vector<uint8_t> data(8 * 40, 0);
      auto g = GgufFile::parse(forge({{"blk.0.ffn_up.weight", {256, 1}, t, data}}));
      auto e = expect_throw<GgufError>([&] { Weights::load(g, 0); });
      CHECK(e.kind == GgufError::Unsupported);
    }
  });
  run("truncated_tensor_is_range_error", [] {
    auto bytes = forge({{"w", {256, 2}, 12, rand_blocks(12, 2)}});
    bytes.resize(bytes.size() - 10);
    auto g = GgufFile::parse(bytes);
    size_t len;
    auto e = expect_throw<GgufError>([&] { g.tensor_bytes(g.tensors[0], &len); });
    CHECK(e.kind == GgufError::Range);
  });
  run("fp8_weight_creation_checks_shapes", [] {  // fp8_weight.rs:104-115, 17-40
    auto f = Fp8Weight::create(Tensor::meta({4, 8}, DType::F8E4M3), Tensor::meta({4}, DType::F32), 8, 4);
    CHECK(f.in_dim() == 8 && f.out_dim() == 4 && f.resident_bytes() == 4 * 8 + 4 * 4);
    Fp8Weight::create(Tensor::meta({4, 8}, DType::F8E4M3), Tensor::meta({4, 1}, DType::F32), 8, 4);
    auto e = expect_throw<ModelError>([] {
      Fp8Weight::create(Tensor::meta({8, 4}, DType::F8E4M3), Tensor::meta({4}, DType::F32), 8, 4);
    });
    CHECK(e.kind == ModelError::Shape && e.name == "fp8_weight");
    auto e2 = expect_throw<ModelError>([] {
      Fp8Weight::create(Tensor::meta({4, 8}, DType::F8E4M3), Tensor::meta({3}, DType::F32), 8, 4);
    });
    CHECK(e2.kind == ModelError::Shape && e2.name == "fp8_scale");
  });
  run("missing_weight", [] {
    auto w = Weights::from_parts(0, {});
    auto e = expect_throw<ModelError>([&] { w.linear(Tensor::meta({1, 4}, DType::F32), "nope"); });
    CHECK(e.kind == ModelError::MissingWeight);
    CHECK(!w.contains_key("nope"));
  });
}

// ----------------------------------------------------------------- GPU ------

static std::vector<uint8_t> q8_rows(const std::vector<std::vector<int>> &rows) {
  std::vector<uint8_t> b;
  for (const auto &r : rows) {
    b.push_back(0x00);
    b.push_back(0x3C);  // d = 1.0
    for (int i = 0; i < 32; ++i) b.push_back((uint8_t)(int8_t)(i < (int)r.size() ? r[i] : 0));
  }
  return b;
}

static void gpu_tests() {
  run("linear_dense_and_quantized", [] {  // linear_layer.rs:129-140
    auto blocks = q8_rows({{1, 2, 3}, {4, 5, 6}});
    std::unordered_map<std::string, std::shared_ptr<QMatMul>> q;
    q["quant.weight"] = std::make_shared<QMatMul>(8, blocks.data(), blocks.size(), 2, 32, 0);
    auto w = Weights::from_quantized(0, {}, q);
    std::vector<float> xv(32, 0.0f);
    xv[0] = xv[1] = xv[2] = 1.0f;
    auto x = Tensor::from_host(xv.data(), {1, 32}, DType::F32, 0);
    auto y = w.linear(x, "quant.weight");
    CHECK((y.dims() == std::vector<size_t>{1, 2}));
    auto v = y.to_vec<float>();
    CHECK(v[0] == 6.0f && v[1] == 15.0f);
    auto bad = Tensor::from_host(xv.data(), {1, 16}, DType::F32, 0);
    auto e = expect_throw<ModelError>([&] { w.linear(bad, "quant.weight"); });
    CHECK(e.kind == ModelError::Shape);
  });
  run("embed_dense_and_quantized", [] {  // embed_layer.rs:92-125, rows 32 wide
    std::vector<std::vector<int>> rows;
    std::vector<float> dense;
    for (int r = 0; r < 4; ++r) {
      std::vector<int> q;
      for (int i = 0; i < 32; ++i) q.push_back(3 * r + i);
      rows.push_back(q);
      for (int i = 0; i < 32; ++i) dense.push_back((float)(3 * r + i));
    }
    auto blocks = q8_rows(rows);
    std::unordered_map<std::string, Tensor> map;
    map["dense_embd"] = Tensor::from_host(dense.data(), {4, 32}, DType::F32, 0);
    auto w = Weights::from_quantized(0, map, {{"quant_embd", std::make_shared<QMatMul>(8, blocks.data(), blocks.size(), 4, 32, 0)}});
    const std::vector<uint32_t> ids = {1, 3};
    auto od = w.embed("dense_embd", ids), oq = w.embed("quant_embd", ids);
    CHECK((od.dims() == std::vector<size_t>{1, 2, 32}) && (oq.dims() == std::vector<size_t>{1, 2, 32}));
    auto dv = od.to_vec<float>(), qv = oq.to_vec<float>();
    CHECK(dv[0] == 3.0f && dv[1] == 4.0f && dv[2] == 5.0f && dv[32] == 9.0f && dv[33] == 10.0f && dv[34] == 11.0f);
    CHECK(std::memcmp(dv.data(), qv.data(), dv.size() * 4) == 0);
    auto cand = w.candidate_weights("quant_embd", ids);
    CHECK((cand.dims() == std::vector<size_t>{2, 32}));
    CHECK((w.embed("quant_embd", {}).dims() == std::vector<size_t>{1, 0, 32}));
    auto e = expect_throw<ModelError>([&] { w.embed("quant_embd", {4}); });
    CHECK(e.kind == ModelError::Shape);
    auto m = expect_throw<ModelError>([&] { w.embed("nope", ids); });
    CHECK(m.kind == ModelError::MissingWeight);
  });
  run("weights_from_quantized_resident_bytes", [] {  // store.rs:231-243
    auto blocks = q8_rows({{1}, {2}, {3}, {4}});
    auto qm = std::make_shared<QMatMul>(8, blocks.data(), blocks.size(), 4, 32, 0);
    auto w = Weights::from_quantized(0, {}, {{"q1", qm}, {"q2_alias", qm}});
    CHECK(w.contains_key("q1") && w.contains_key("q2_alias"));
    CHECK(w.resident_bytes() == qm->storage_size_in_bytes());
  });
  run("get_dequantizes_bit_exact", [] {
    for (uint32_t t : {8u, 12u, 14u}) {
      size_t elems, bytes;
      rqo_block_geometry(t, &elems, &bytes);
      const size_t n = 6, k = 896;
      auto blocks = rand_blocks(t, n * k / elems);
      auto w = Weights::from_quantized(0, {}, {{"w", std::make_shared<QMatMul>((int)t, blocks.data(), blocks.size(), n, k, 0)}});
      auto got = w.get("w").to_vec<float>();
      std::vector<float> want(n * k);
      CHECK(rqo_dequant_tensor(t, blocks.data(), blocks.size(), n * k, want.data()) == 0);
      CHECK(std::memcmp(got.data(), want.data(), want.size() * 4) == 0);
    }
  });
  run("load_gguf_and_linear", [] {  // load_gguf.rs:40-120 on a forged file
    const size_t k = 512, n4 = 64, n6 = 48;
    auto b4 = rand_blocks(12, n4 * k / 256), b6 = rand_blocks(14, n6 * k / 256);
    auto g = GgufFile::parse(forge({{"blk.0.ffn_gate.weight", {k, n4}, 12, b4},
                                    {"blk.0.attn_v.weight", {k, n6}, 14, b6},
                                    {"token_embd.weight", {k, n4}, 12, b4}}));
    auto w = Weights::load(g, 0);
    CHECK(w.q_matmul("output.weight") == w.q_matmul("token_embd.weight"));  // tied head
    for (const char *name : {"blk.0.ffn_gate.weight", "blk.0.attn_v.weight"}) {
      const bool six = std::string(name).find("attn_v") != std::string::npos;
      const size_t n = six ? n6 : n4;
      auto &blk = six ? b6 : b4;
      std::vector<float> wf(n * k);
      CHECK(rqo_dequant_tensor(six ? 14 : 12, blk.data(), blk.size(), n * k, wf.data()) == 0);
      for (size_t m : {1, 3}) {
        auto xv = rand_normal(m * k);
        auto y = w.linear(Tensor::from_host(xv.data(), {m, k}, DType::F32, 0), name);
        CHECK((y.dims() == std::vector<size_t>{m, n}));
        std::vector<double> r(m * n);
        rqo_linear_f64(xv.data(), (int64_t)m, wf.data(), (int64_t)n, (int64_t)k, r.data());
        CHECK(norm_err(y.to_vec<float>(), r) <= 1e-3);
      }
    }
  });
  run("load_gguf_one_dim_block_tensor_as_f32", [] {  // load_gguf.rs:107-110: tensor_f32
    // a block-format tensor that is not 2-D is decoded to dense f32, as the
    // reference's tensor_f32 does, bit-exact against the oracle
    auto b8 = rand_blocks(8, 16);
    auto g = GgufFile::parse(forge({{"blk.0.attn_norm.weight", {512}, 8, b8}}));
    auto w = Weights::load(g, 0);
    CHECK(w.q_matmul("blk.0.attn_norm.weight") == nullptr);
    auto got = w.get("blk.0.attn_norm.weight");
    CHECK((got.dims() == std::vector<size_t>{512}) && got.dtype() == DType::F32);
    std::vector<float> want(512);
    CHECK(rqo_dequant_tensor(8, b8.data(), b8.size(), 512, want.data()) == 0);
    auto v = got.to_vec<float>();
    CHECK(std::memcmp(v.data(), want.data(), want.size() * 4) == 0);
  });
  run("cpu_fp8_gemm_matches_reference", [] {  // fp8_gemm.rs:198-208, on the device
    std::vector<float> xv{1, 2, 3, 4};
    std::vector<uint8_t> wv{0x38, 0x00, 0x00, 0x40};
    std::vector<float> sv{2.0f, 0.5f};
    auto x = Tensor::from_host(xv.data(), {2, 2}, DType::F32, 0);
    auto w = Tensor::from_host(wv.data(), {2, 2}, DType::F8E4M3, 0);
    auto s = Tensor::from_host(sv.data(), {2}, DType::F32, 0);
    auto y = HipSubstrate().fp8_gemm(x, w, &s);
    CHECK((y.dims() == std::vector<size_t>{2, 2}));
    CHECK((y.to_vec<float>() == std::vector<float>{2, 2, 6, 4}));
  });
  run("fp8_weight_forward_matches_dequant", [] {  // fp8_weight.rs:117-133
    std::vector<uint8_t> wv{0x38, 0x40, 0x30, 0x44};  // 1.0, 2.0, 0.5, 3.0
    std::vector<float> sv{2.0f, 0.5f}, xv{1.5f, -2.0f};
    auto f = Fp8Weight::create(Tensor::from_host(wv.data(), {2, 2}, DType::F8E4M3, 0),
                               Tensor::from_host(sv.data(), {2}, DType::F32, 0), 2, 2);
    auto out = f.forward(Tensor::from_host(xv.data(), {1, 2}, DType::F32, 0), HipSubstrate()).to_vec<float>();
    const float expected[2] = {1.5f * 2.0f * 1.0f - 2.0f * 2.0f * 2.0f, 1.5f * 0.5f * 0.5f - 2.0f * 0.5f * 3.0f};
    for (int i = 0; i < 2; ++i) CHECK(std::fabs(out[i] - expected[i]) < 1e-3f);
  });
  run("linear_fp8_cuda", [] {  // linear_layer.rs:187-210
    std::vector<uint8_t> wb(16 * 16, 0x38);
    std::unordered_map<std::string, Tensor> map;
    map["w"] = Tensor::from_host(wb.data(), {16, 16}, DType::F8E4M3, 0);
    auto weights = Weights::from_parts(0, map);
    std::vector<float> ones(16, 1.0f);
    auto x = Tensor::from_host(ones.data(), {1, 16}, DType::F32, 0);
    auto y = weights.linear(x, "w");
    CHECK((y.dims() == std::vector<size_t>{1, 16}));
    for (float v : y.to_vec<float>()) CHECK(std::fabs(v - 16.0f) < 1e-1f);
    std::vector<float> sv(16);
    for (int i = 0; i < 16; ++i) sv[i] = (float)(i + 1);
    map["w.scale"] = Tensor::from_host(sv.data(), {16}, DType::F32, 0);
    auto weights2 = Weights::from_parts(0, map);
    auto vals = weights2.linear(x, "w").to_vec<float>();
    for (int i = 0; i < 16; ++i) CHECK(std::fabs(vals[i] - 16.0f * sv[i]) < 1e-1f);
  });
  run("marlin_gemv_matches_dequant", [] {  // marlin_gemv.rs:209-222
    const float wv[8] = {1.0f, -2.0f, 3.0f, 0.0f, 0.5f, 1.5f, -0.5f, 2.0f};
    const float sv[2] = {0.5f, 0.25f};
    auto w = Tensor::from_host(wv, {2, 4}, DType::F32, 0);
    auto sc = Tensor::from_host(sv, {2}, DType::F32, 0);
    auto mw = repack_marlin_tiles(w, sc);
    CHECK(mw.resident_bytes() == (2 * 4) * 4 + 2 * 4);
    uint32_t want[8];
    rqo_marlin_repack(wv, sv, 2, 4, want);
    auto got = mw.packed().to_vec<uint32_t>();
    CHECK(got.size() == 8 && std::memcmp(got.data(), want, sizeof(want)) == 0);
    const float xv[4] = {2.0f, 1.0f, -1.0f, 3.0f};
    auto x = Tensor::from_host(xv, {1, 4}, DType::F32, 0);
    auto y = HipSubstrate().marlin_gemv(x, mw).to_vec<float>();
    auto deq = mw.dequantize().to_vec<float>();
    for (int r = 0; r < 2; ++r) {
      float e = 0.0f;
      for (int k = 0; k < 4; ++k) e += xv[k] * deq[r * 4 + k];
      CHECK(std::fabs(y[r] - e) < 1e-4f);
    }
    CHECK(y[0] == -3.0f && y[1] == 8.25f);
  });
  run("linear_marlin", [] {  // linear_layer.rs:143-160
    const float wv[8] = {1, 2, 3, 4, 2, 3, 4, 5};
    const float ones[80] = {1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                            1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                            1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1};
    auto mw = repack_marlin_tiles(Tensor::from_host(wv, {2, 4}, DType::F32, 0),
                                  Tensor::from_host(ones, {2}, DType::F32, 0));
    auto weights = Weights::from_parts(0, {});
    weights.insert_marlin("blk.0.attn_q", mw);
    auto y = weights.linear(Tensor::from_host(ones, {1, 4}, DType::F32, 0), "blk.0.attn_q.weight");
    CHECK((y.dims() == std::vector<size_t>{1, 2}));
    auto v = y.to_vec<float>();
    CHECK(v[0] == 10.0f && v[1] == 14.0f);
    auto bad = Tensor::from_host(ones, {1, 80}, DType::F32, 0);
    auto e = expect_throw<ModelError>([&] { weights.linear(bad, "blk.0.attn_q.weight"); });
    CHECK(e.kind == ModelError::Shape);
  });
  run("linear_bias_quantized_and_fp8", [] {  // linear_layer.rs:107-118
    // Quantized: the bias (F16, as the CUDA store keeps dense tensors) rides
    // in the kernel's epilogue; FP8: linear, then the broadcast add.
    auto blocks = q8_rows({{1, 2, 3}, {4, 5, 6}});
    const _Float16 bh[2] = {(_Float16)0.5f, (_Float16)-2.0f};
    std::vector<uint8_t> wb(2 * 32, 0x38);  // e4m3 1.0
    std::unordered_map<std::string, Tensor> map;
    map["b"] = Tensor::from_host(bh, {2}, DType::F16, 0);
    map["f8"] = Tensor::from_host(wb.data(), {2, 32}, DType::F8E4M3, 0);
    auto w = Weights::from_quantized(0, map, {{"q", std::make_shared<QMatMul>(8, blocks.data(), blocks.size(), 2, 32, 0)}});
    std::vector<float> xv(64, 0.0f);
    xv[0] = xv[1] = xv[2] = 1.0f;        // row 0: [6, 15] before the bias
    xv[32] = 2.0f;                        // row 1: [2, 8]
    auto x = Tensor::from_host(xv.data(), {2, 32}, DType::F32, 0);
    const std::string bname = "b";
    auto yq = w.linear_bias(x, "q", &bname).to_vec<float>();
    CHECK((yq == std::vector<float>{6.5f, 13.0f, 2.5f, 6.0f}));
    CHECK((w.linear_bias(x, "q", nullptr).to_vec<float>() == std::vector<float>{6, 15, 2, 8}));
    auto y8 = w.linear_bias(x, "f8", &bname).to_vec<float>();  // sum of x + bias
    CHECK((y8 == std::vector<float>{3.5f, 1.0f, 2.5f, 0.0f}));
    const std::string missing = "nope";
    auto e = expect_throw<ModelError>([&] { w.linear_bias(x, "q", &missing); });
    CHECK(e.kind == ModelError::MissingWeight);
  });
  run("fp8_scale_bf16_per_row_and_per_tensor", [] {  // fp8_gemm.rs: the scale is read as F32
    std::vector<uint8_t> wv{0x38, 0x00, 0x00, 0x40};  // [[1, 0], [0, 2]]
    std::vector<float> xv{1, 2, 3, 4};
    auto x = Tensor::from_host(xv.data(), {2, 2}, DType::F32, 0);
    auto w = Tensor::from_host(wv.data(), {2, 2}, DType::F8E4M3, 0);
    const uint16_t row_bf16[2] = {0x4000, 0x3F00};  // 2.0, 0.5
    auto s_row = Tensor::from_host(row_bf16, {2}, DType::BF16, 0);
    CHECK((HipSubstrate().fp8_gemm(x, w, &s_row).to_vec<float>() == std::vector<float>{2, 2, 6, 4}));
    const uint16_t one_bf16[1] = {0x4040};  // 3.0
    auto s_one = Tensor::from_host(one_bf16, {1}, DType::BF16, 0);
    CHECK((HipSubstrate().fp8_gemm(x, w, &s_one).to_vec<float>() == std::vector<float>{3, 12, 9, 24}));
    auto f = Fp8Weight::create(w, s_row, 2, 2);
    CHECK(f.resident_bytes() == 4 + 2 * 2);  // the scale keeps its dtype (fp8_weight.rs:63-66)
    CHECK((f.forward(x, HipSubstrate()).to_vec<float>() == std::vector<float>{2, 2, 6, 4}));
  });
  run("cuda_fp8_gemm_runs_or_skips", [] {  // fp8_gemm.rs:209-230
    std::vector<uint8_t> xb(16 * 16, 0x38), wb(16 * 16, 0x38);
    std::vector<float> sv(16);
    for (int i = 0; i < 16; ++i) sv[i] = (float)(i + 1);
    auto x = Tensor::from_host(xb.data(), {16, 16}, DType::F8E4M3, 0);
    auto w = Tensor::from_host(wb.data(), {16, 16}, DType::F8E4M3, 0);
    auto s = Tensor::from_host(sv.data(), {16}, DType::F32, 0);
    auto y = HipSubstrate().fp8_gemm(x, w, &s);
    CHECK((y.dims() == std::vector<size_t>{16, 16}) && y.dtype() == DType::F16);
    auto raw = y.to_vec<_Float16>();
    for (int r = 0; r < 16; ++r)
      for (int c = 0; c < 16; ++c) CHECK(std::fabs((float)raw[r * 16 + c] - 16.0f * sv[c]) < 1e-1f);
  });
}

int main(int argc, char **argv) {
  const bool cpu = argc < 2 || std::strcmp(argv[1], "--gpu") != 0;
  if (cpu) cpu_tests();
  else gpu_tests();
  std::printf("%d/%d passed\n", g_run - g_fail, g_run);
  return g_fail ? 1 : 0;
}
