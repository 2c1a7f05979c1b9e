// kiln_host_run — drives the C++ host layer (kiln_amd/host) for the tests.
//
//   kiln_host_run selftest            checks that need no GPU (JSON reader,
//                                     config validation, error paths)
//   kiln_host_run job <job.json>      loads a checkpoint directory and runs one
//                                     layer call on the GPU, writing raw output
//
// job.json: {"model_dir": d, "op": "linear"|"mlp"|"embed"|"as_linear"|"probe"|"load"|"load_all"|"switch",
//            "prefix": p, "input": file, "input_shape": [...],
//            "input_dtype": "bfloat16"|"float16"|"float32"|"uint32"|"int32",
//            "output": file}
// It prints one JSON line: {"ok": true, "shape": [...], "dtype": ...} or
// {"ok": false, "error": "..."}; "probe" prints {"ok": true, "m": first
// divergent M}; "load" prints the linear's io_features and remaining tensors.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>

#include "../../kiln_amd/host/kiln_host.hpp"

using namespace kiln;

static int fails = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      ++fails;                                                        \
    }                                                                 \
  } while (0)

static std::string jstr(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') o += '\\';
    if (c == '\n') {
      o += "\\n";
      continue;
    }
    o += c;
  }
  return o + "\"";
}

static int selftest() {
  // JSON reader
  auto v = json::parse(R"({"a": [1, 2.5, -3e2], "b": {"c": "x\"yé"}, "t": true, "n": null})");
  CHECK(v.is_object());
  CHECK(v.get("a")->arr.size() == 3 && v.get("a")->arr[2].num == -300.0);
  CHECK(v.get("b")->get("c")->str == "x\"y\xc3\xa9");
  CHECK(v.get("t")->b && v.get("n")->kind == json::Value::Null);
  bool threw = false;
  try {
    json::parse("{\"a\": [1, 2}");
  } catch (const std::exception&) {
    threw = true;
  }
  CHECK(threw);

  // config validation (crates/kiln-models/src/config.rs:137-148, 735-760)
  CHECK(validate_quant_params(Quantization{64, 4}).ok());
  CHECK(validate_quant_params(Quantization{128, 8}).ok());
  auto bad = validate_quant_params(Quantization{64, 3});
  CHECK(!bad.ok() && bad.error().message.find("bits=3 group_size=64") != std::string::npos);
  CHECK(!validate_quant_params(Quantization{48, 4}).ok());
  CHECK(validate_quant_params(std::nullopt).ok());
  auto mode = validate_quantization(json::parse(R"({"quantization": {"group_size": 64, "bits": 4, "mode": "mxfp4"}})"));
  CHECK(!mode.ok() && mode.error().message.find("\"mxfp4\"") != std::string::npos);
  auto over = validate_quantization(json::parse(
      R"({"quantization": {"group_size": 64, "bits": 4, "model.layers.0.mlp": {"bits": 8}, "a": 1}})"));
  CHECK(!over.ok() && over.error().message.find("[\"a\", \"model.layers.0.mlp\"]") != std::string::npos);
  auto q = quantization_from_config(json::parse(R"({"quantization": {"group_size": 32, "bits": 8}})"));
  CHECK(q.ok() && q.value() && q.value()->group_size == 32 && q.value()->bits == 8);
  auto none = quantization_from_config(json::parse(R"({"hidden_size": 8})"));
  CHECK(none.ok() && !none.value());
  auto domain = quantization_from_config(json::parse(R"({"quantization": {"group_size": 16, "bits": 4}})"));
  CHECK(!domain.ok());

  // missing checkpoint is an error, not an abort
  auto store = WeightStore::from_model_dir("/nonexistent-kiln-dir", Stream::gpu());
  CHECK(!store.ok() && store.error().message.find("failed to read") != std::string::npos);

  // dtype sizes
  CHECK(dtype_size(Dtype::Bfloat16) == 2 && dtype_size(Dtype::Uint32) == 4);

  // safetensors header validation: malformed headers are errors
  auto st_file = [](const std::string& header, size_t data_bytes) {
    std::string f(8, '\0');
    const uint64_t n = header.size();
    std::memcpy(&f[0], &n, 8);
    return f + header + std::string(data_bytes, '\x01');
  };
  auto hdr = [&](const std::string& h, size_t data_bytes) {
    const std::string f = st_file(h, data_bytes);
    return read_safetensors_header(f.data(), f.size(), "t.safetensors");
  };
  auto okh = hdr(R"({"a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [0, 12]}, "__metadata__": {}})", 12);
  CHECK(okh.ok() && okh.value().size() == 1 && okh.value()[0].nbytes == 12 && okh.value()[0].shape[1] == 3);
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [-2, 3], "data_offsets": [0, 12]}})", 12).ok());
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [2.5, 3], "data_offsets": [0, 12]}})", 12).ok());
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [4294967296, 4294967296, 4294967296], "data_offsets": [0, 12]}})", 12).ok());
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [0, 14]}})", 14).ok());   // shape mismatch
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [0, 12]}})", 8).ok());    // past the end
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [12, 0]}})", 12).ok());
  CHECK(!hdr(R"({"a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [-1e300, 12]}})", 12).ok());
  CHECK(!hdr(R"({"a": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}})", 8).ok());
  {
    std::string f = st_file("{}", 0);
    const uint64_t huge = ~uint64_t(0) - 3;
    std::memcpy(&f[0], &huge, 8);
    CHECK(!read_safetensors_header(f.data(), f.size(), "t").ok());
  }
  // an array too large for any device is an error, not a hang
  CHECK(!Array::empty({int64_t(1) << 40, int64_t(1) << 20}, Dtype::Float32, Stream::gpu()).ok());

  std::printf("{\"ok\": %s, \"failures\": %d}\n", fails ? "false" : "true", fails);
  return fails ? 1 : 0;
}

static Dtype parse_dtype(const std::string& s) {
  if (s == "bfloat16") return Dtype::Bfloat16;
  if (s == "float16") return Dtype::Float16;
  if (s == "float32") return Dtype::Float32;
  if (s == "uint32") return Dtype::Uint32;
  return Dtype::Int32;
}

// A field of /proc/self/status in KiB (VmRSS: resident now; VmHWM: peak).
static long proc_kib(const char* key) {
  std::ifstream f("/proc/self/status");
  std::string line;
  while (std::getline(f, line))
    if (line.compare(0, std::strlen(key), key) == 0) return std::atol(line.c_str() + std::strlen(key));
  return -1;
}

static int fail_json(const std::string& msg) {
  std::printf("{\"ok\": false, \"error\": %s}\n", jstr(msg).c_str());
  return 2;
}

static int job(const std::string& path) {
  std::ifstream f(path);
  std::stringstream ss;
  ss << f.rdbuf();
  json::Value j = json::parse(ss.str());
  const std::string dir = j.get("model_dir")->str, op = j.get("op")->str, prefix = j.get("prefix")->str;
  Stream s = Stream::gpu();

  std::ifstream cf(dir + "/config.json");
  std::stringstream cs;
  cs << cf.rdbuf();
  auto quant = quantization_from_config(json::parse(cs.str()));
  if (!quant) return fail_json(quant.error().message);
  if (op == "load_all") (void)hipFree(nullptr);  // the runtime is up before memory is measured
  const long rss_before = proc_kib("VmRSS:");
  auto store = WeightStore::from_model_dir(dir, s);
  if (!store) return fail_json(store.error().message);
  if (op == "load_all") {  // the whole store: host memory around the load, and
                           // FNV-1a hashes of each tensor's first and last 4 KiB
    const long hwm_after = proc_kib("VmHWM:");
    std::string hs = "{";
    for (const auto& name : store.value().remaining()) {
      auto t = store.value().take(name);
      if (!t) return fail_json(t.error().message);
      const Array& a = t.value();
      const size_t n = a.nbytes(), k = n < 4096 ? n : 4096;
      std::vector<unsigned char> h(2 * k);
      if (k && (hipMemcpy(h.data(), a.data(), k, hipMemcpyDeviceToHost) != hipSuccess ||
                hipMemcpy(h.data() + k, static_cast<const char*>(a.data()) + n - k, k, hipMemcpyDeviceToHost) !=
                    hipSuccess))
        return fail_json("readback of " + name);
      uint64_t f = 1469598103934665603ull;
      for (unsigned char c : h) f = (f ^ c) * 1099511628211ull;
      hs += (hs.size() > 1 ? ", " : "") + jstr(name) + ": " + jstr(std::to_string(f));
    }
    std::printf("{\"ok\": true, \"rss_before_kib\": %ld, \"hwm_after_kib\": %ld, \"hashes\": %s}}\n",
                rss_before, hwm_after, hs.c_str());
    return 0;
  }

  if (op == "load") {
    auto l = nn::Linear::load(store.value(), prefix, quant.value());
    if (!l) return fail_json(l.error().message);
    auto io = l.value().io_features();
    std::string rem = "[";
    for (const auto& n : store.value().remaining()) rem += (rem.size() > 1 ? ", " : "") + jstr(n);
    std::printf("{\"ok\": true, \"in\": %lld, \"out\": %lld, \"quantized\": %s, \"remaining\": %s]}\n",
                (long long)io.first, (long long)io.second, l.value().quantized() ? "true" : "false",
                rem.c_str());
    return 0;
  }

  std::vector<int64_t> shape;
  for (const auto& d : j.get("input_shape")->arr) shape.push_back((int64_t)d.num);
  std::ifstream inf(j.get("input")->str, std::ios::binary);
  std::string in((std::istreambuf_iterator<char>(inf)), std::istreambuf_iterator<char>());
  auto x = Array::from_bytes(in.data(), in.size(), shape, parse_dtype(j.get("input_dtype")->str), s);
  if (!x) return fail_json(x.error().message);

  Result<Array> y = Error{"unknown op " + op};
  if (op == "switch") {  // SwitchLinear: prefix = the MLP prefix, plus proj, experts, ids
    std::vector<int64_t> ishape;
    for (const auto& d : j.get("ids_shape")->arr) ishape.push_back((int64_t)d.num);
    std::ifstream idf(j.get("ids")->str, std::ios::binary);
    std::string ib((std::istreambuf_iterator<char>(idf)), std::istreambuf_iterator<char>());
    auto ids = Array::from_bytes(ib.data(), ib.size(), ishape, Dtype::Uint32, s);
    if (!ids) return fail_json(ids.error().message);
    auto sl = nn::SwitchLinear::load(store.value(), prefix, j.get("proj")->str, (int)j.get("experts")->num,
                                     quant.value(), s);
    if (!sl) return fail_json(sl.error().message);
    y = sl.value().forward(x.value(), ids.value(), j.get("sorted") && j.get("sorted")->b, s);
  } else if (op == "mlp") {  // Mlp: prefix = the MLP prefix; "activation": "silu" | "gelu_approx"
    const auto* act = j.get("activation");
    const nn::Activation a = act && act->str == "gelu_approx" ? nn::Activation::GeluApprox : nn::Activation::Silu;
    auto m = nn::Mlp::load(store.value(), prefix, quant.value(), a);
    if (!m) return fail_json(m.error().message);
    y = m.value().forward(x.value(), s);
  } else if (op == "linear") {
    auto l = nn::Linear::load(store.value(), prefix, quant.value());
    if (!l) return fail_json(l.error().message);
    y = l.value().forward(x.value(), s);
  } else if (op == "embed" || op == "as_linear" || op == "probe") {
    auto e = nn::Embedding::load(store.value(), prefix, quant.value());
    if (!e) return fail_json(e.error().message);
    if (op == "embed") {
      y = e.value().lookup(x.value(), s);
    } else if (op == "as_linear") {
      y = e.value().as_linear(x.value(), s);
    } else {
      const nn::Embedding& emb = e.value();
      auto m = nn::probe_row_stability((int64_t)j.get("k")->num, x.value(), s,
                                       [&](const Array& xx) { return emb.as_linear(xx, s); });
      if (!m) return fail_json(m.error().message);
      std::printf("{\"ok\": true, \"m\": %d}\n", m.value());
      return 0;
    }
  }
  if (!y) return fail_json(y.error().message);
  auto bytes = y.value().to_bytes(s);
  if (!bytes) return fail_json(bytes.error().message);
  std::ofstream of(j.get("output")->str, std::ios::binary);
  of.write(reinterpret_cast<const char*>(bytes.value().data()), (std::streamsize)bytes.value().size());
  std::string sh = "[";
  for (int i = 0; i < y.value().ndim(); ++i) sh += (i ? ", " : "") + std::to_string(y.value().dim(i));
  std::printf("{\"ok\": true, \"shape\": %s], \"dtype\": \"%s\"}\n", sh.c_str(), dtype_name(y.value().dtype()));
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && std::strcmp(argv[1], "selftest") == 0) return selftest();
  if (argc >= 3 && std::strcmp(argv[1], "job") == 0) {
    try {
      return job(argv[2]);
    } catch (const std::exception& e) {
      return fail_json(e.what());
    }
  }
  std::fprintf(stderr, "usage: kiln_host_run selftest | job <job.json>\n");
  return 64;
}
