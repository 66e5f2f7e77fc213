// A C++ caller of the drop-in API, built without Python: what an engine that
// links csrc/torch_api/{torch_api,registry}.cpp and libxk.so sees.  It follows
// the reference gtests' flow (triton_npu/test/triton_chunk_gated_delta_rule_
// test.cpp:330-340: make a device tensor, register the kernel by name, check
// its stub; then :190-323: call the torch-level op), on the committed golden
// inputs, and writes the outputs to a safetensors file that the Python test
// compares with the golden outputs.
//
//   xk_api_consumer --registry                 registry checks only (no GPU)
//   xk_api_consumer <golden.safetensors> <out.safetensors>
//
// Ops called (xllm::kernel::npu, triton_ops_api.h): layer_norm_fwd on the
// golden case "layer_norm_gated" and npu_chunk_gated_delta_rule on "gdn_chunk".
#include <torch/torch.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernel_registry.h"
#include "triton_ops_api.h"

namespace npu = xllm::kernel::npu;

namespace {

// ---------------------------------------------------------------------------
// safetensors: an 8-byte little-endian header length, a JSON header mapping
// each tensor name to {"dtype", "shape", "data_offsets"} (plus an optional
// "__metadata__" object), then the raw little-endian data.
// ---------------------------------------------------------------------------
struct Json {
  enum Kind { kNull, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;
};

class Parser {
 public:
  explicit Parser(const std::string& s) : s_(s) {}
  Json parse() {
    Json v = value();
    ws();
    if (i_ != s_.size()) throw std::runtime_error("trailing bytes in safetensors header");
    return v;
  }

 private:
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t'))
      ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) throw std::runtime_error("truncated safetensors header");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) throw std::runtime_error(std::string("safetensors header: expected ") + c);
    ++i_;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\') {
        ++i_;
        if (i_ >= s_.size()) break;
      }
      out += s_[i_++];
    }
    expect('"');
    return out;
  }
  Json value() {
    Json v;
    const char c = peek();
    if (c == '{') {
      v.kind = Json::kObj;
      ++i_;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      while (true) {
        std::string k = string();
        expect(':');
        v.obj[k] = value();
        if (peek() == ',') {
          ++i_;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      v.kind = Json::kArr;
      ++i_;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      while (true) {
        v.arr.push_back(value());
        if (peek() == ',') {
          ++i_;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = Json::kStr;
      v.str = string();
      return v;
    }
    const size_t b = i_;
    while (i_ < s_.size() && (isdigit(s_[i_]) || s_[i_] == '-' || s_[i_] == '+' || s_[i_] == '.' ||
                              s_[i_] == 'e' || s_[i_] == 'E'))
      ++i_;
    if (b == i_) throw std::runtime_error("safetensors header: bad value");
    v.kind = Json::kNum;
    v.num = std::stod(s_.substr(b, i_ - b));
    return v;
  }
  const std::string& s_;
  size_t i_ = 0;
};

torch::ScalarType dtype_of(const std::string& d) {
  if (d == "F32") return torch::kFloat32;
  if (d == "BF16") return torch::kBFloat16;
  if (d == "F16") return torch::kFloat16;
  if (d == "I32") return torch::kInt32;
  if (d == "I64") return torch::kInt64;
  throw std::runtime_error("unsupported safetensors dtype " + d);
}

const char* name_of(torch::ScalarType t) {
  switch (t) {
    case torch::kFloat32: return "F32";
    case torch::kBFloat16: return "BF16";
    case torch::kInt32: return "I32";
    case torch::kInt64: return "I64";
    default: throw std::runtime_error("unsupported dtype for safetensors output");
  }
}

std::map<std::string, torch::Tensor> load_safetensors(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  uint64_t n = 0;
  f.read(reinterpret_cast<char*>(&n), 8);
  std::string hdr(n, '\0');
  f.read(&hdr[0], static_cast<std::streamsize>(n));
  std::stringstream rest;
  rest << f.rdbuf();
  const std::string data = rest.str();
  const Json h = Parser(hdr).parse();
  std::map<std::string, torch::Tensor> out;
  for (const auto& kv : h.obj) {
    if (kv.first == "__metadata__") continue;
    const Json& e = kv.second;
    std::vector<int64_t> shape;
    for (const Json& d : e.obj.at("shape").arr) shape.push_back(static_cast<int64_t>(d.num));
    const auto& off = e.obj.at("data_offsets").arr;
    const size_t a = static_cast<size_t>(off.at(0).num), b = static_cast<size_t>(off.at(1).num);
    auto t = torch::empty(shape, torch::TensorOptions().dtype(dtype_of(e.obj.at("dtype").str)));
    if (b < a || b > data.size() || static_cast<size_t>(t.nbytes()) != b - a)
      throw std::runtime_error("safetensors entry " + kv.first + " has inconsistent offsets");
    std::memcpy(t.data_ptr(), data.data() + a, b - a);
    out[kv.first] = t;
  }
  return out;
}

void save_safetensors(const std::string& path, const std::map<std::string, torch::Tensor>& ts) {
  std::ostringstream hdr;
  hdr << "{";
  size_t off = 0;
  bool first = true;
  std::vector<torch::Tensor> order;
  for (const auto& kv : ts) {
    const torch::Tensor t = kv.second.contiguous().cpu();
    order.push_back(t);
    hdr << (first ? "" : ",") << "\"" << kv.first << "\":{\"dtype\":\"" << name_of(t.scalar_type())
        << "\",\"shape\":[";
    for (int64_t d = 0; d < t.dim(); ++d) hdr << (d ? "," : "") << t.size(d);
    hdr << "],\"data_offsets\":[" << off << "," << off + t.nbytes() << "]}";
    off += t.nbytes();
    first = false;
  }
  hdr << "}";
  std::string h = hdr.str();
  while (h.size() % 8) h += ' ';
  std::ofstream f(path, std::ios::binary);
  const uint64_t n = h.size();
  f.write(reinterpret_cast<const char*>(&n), 8);
  f.write(h.data(), static_cast<std::streamsize>(h.size()));
  for (const auto& t : order) f.write(static_cast<const char*>(t.data_ptr()), t.nbytes());
  if (!f) throw std::runtime_error("cannot write " + path);
}

// Distinct files of the HIP runtime mapped into this process: libxk.so and
// PyTorch must share one (the library names it by soname, libamdhip64.so.7,
// which the runtime PyTorch loads also carries).
std::vector<std::string> hip_runtimes() {
  std::ifstream maps("/proc/self/maps");
  std::vector<std::string> out;
  std::string line;
  while (std::getline(maps, line)) {
    const size_t p = line.find('/');
    if (p == std::string::npos) continue;
    const std::string path = line.substr(p);
    if (path.find("libamdhip64") == std::string::npos) continue;
    bool seen = false;
    for (const auto& s : out) seen |= s == path;
    if (!seen) out.push_back(path);
  }
  return out;
}

// The reference gtests register each kernel by name before calling its op.
bool registered(const char* kernel) {
  auto& reg = npu::KernelRegistry::get_instance();
  return reg.register_kernel(kernel, "") && reg.get_kernel_stub(kernel) != nullptr &&
         reg.is_kernel_registered(kernel);
}

}  // namespace

int main(int argc, char** argv) {
  try {
    const char* kernels[] = {"layer_norm_fwd_kernel", "chunk_gated_delta_rule_fwd_kernel_h_blockdim64"};
    for (const char* k : kernels) {
      if (!registered(k)) {
        std::fprintf(stderr, "kernel %s is not registered\n", k);
        return 1;
      }
    }
    if (npu::KernelRegistry::get_instance().register_kernel("no_such_kernel", "")) {
      std::fprintf(stderr, "an unknown kernel name was accepted\n");
      return 1;
    }
    const auto rt = hip_runtimes();
    if (rt.size() != 1) {
      std::fprintf(stderr, "expected one HIP runtime mapped, found %zu\n", rt.size());
      for (const auto& s : rt) std::fprintf(stderr, "  %s\n", s.c_str());
      return 1;
    }
    if (argc == 2 && std::string(argv[1]) == "--registry") {
      std::printf("registry ok; HIP runtime %s\n", rt[0].c_str());
      return 0;
    }
    if (argc != 3) {
      std::fprintf(stderr, "usage: %s <golden.safetensors> <out.safetensors> | --registry\n",
                   argv[0]);
      return 2;
    }
    auto gold = load_safetensors(argv[1]);
    const auto dev = torch::Device(torch::kCUDA, 0);
    auto in = [&](const std::string& k) { return gold.at(k).to(dev); };
    std::map<std::string, torch::Tensor> out;

    {  // layer_norm_fwd: grouped LayerNorm (group 256), bias, z gate after the norm
      std::printf("layer_norm_gated\n");
      std::fflush(stdout);
      auto x = in("layer_norm_gated/in/x"), w = in("layer_norm_gated/in/w"),
           b = in("layer_norm_gated/in/b"), z = in("layer_norm_gated/in/z");
      torch::Tensor y = npu::layer_norm_fwd(x, w, b, 1e-5, z, 256, true, false);
      out["layer_norm_gated/y"] = y.to(torch::kFloat32);
    }
    {  // npu_chunk_gated_delta_rule: 2 sequences, in-op l2norm, initial + final states
      std::printf("gdn_chunk\n");
      std::fflush(stdout);
      auto q = in("gdn_chunk/in/q"), k = in("gdn_chunk/in/k"), v = in("gdn_chunk/in/v"),
           g = in("gdn_chunk/in/gate"), beta = in("gdn_chunk/in/beta");
      std::optional<torch::Tensor> h0 = in("gdn_chunk/in/h0"), cu = in("gdn_chunk/in/cu");
      auto res = npu::npu_chunk_gated_delta_rule(q, k, v, g, beta, std::nullopt, h0, true, cu,
                                                 false, true);
      out["gdn_chunk/o"] = res.first.to(torch::kFloat32);
      out["gdn_chunk/state"] = res.second.to(torch::kFloat32);
    }
    save_safetensors(argv[2], out);
    std::printf("ok\n");
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
