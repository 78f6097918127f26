// GGUF model loading (host code): the file reader of src/gguf.rs:225-286 and the config mapping of
// Model::load (src/model.rs:713-921) for the decoder families the training step runs (llama, qwen2,
// mistral, qwen2moe, olmoe: RMSNorm, SwiGLU, RoPE, optional QKV bias, optionally tied head, optional mixture of
// experts). Linear weights are uploaded in their GGUF encoding — every type the reference decodes
// (src/gguf.rs:330-505: F32, F16, BF16, Q8_0, Q4_0, Q5_0, Q4_K, Q5_K, Q6_K); the device repack keeps them
// quantized and bit-exact. Norms, biases and the router are widened to F32 from F32 / F16 / BF16.
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

#include "ctx.hpp"

using namespace hos;

namespace {

enum : uint32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_BF16 = 30 };

struct MetaVal {
  uint32_t type = 0;
  uint64_t u = 0;  // integer kinds and bool
  int64_t i = 0;
  double f = 0;
  std::string s;
  bool is_int = false, is_float = false, is_str = false;
};

struct TInfo {
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;
};

struct GgufFile {
  std::vector<uint8_t> buf;
  std::map<std::string, MetaVal> meta;
  std::map<std::string, TInfo> tensors;
  size_t data_offset = 0;

  bool has(const std::string& n) const { return tensors.count(n) != 0; }
  bool meta_u64(const std::string& k, uint64_t* v) const {
    auto it = meta.find(k);
    if (it == meta.end() || !it->second.is_int) return false;
    *v = it->second.u;
    return true;
  }
  bool meta_f32(const std::string& k, float* v) const {
    auto it = meta.find(k);
    if (it == meta.end()) return false;
    if (it->second.is_float)
      *v = (float)it->second.f;
    else if (it->second.is_int)
      *v = (float)it->second.i;
    else
      return false;
    return true;
  }
  std::string meta_str(const std::string& k, const std::string& dflt) const {
    auto it = meta.find(k);
    return (it == meta.end() || !it->second.is_str) ? dflt : it->second.s;
  }
};

// Bounds-checked little-endian reader (truncated or corrupt files become HOS_E_FORMAT).
struct Reader {
  const std::vector<uint8_t>& b;
  size_t pos = 0;
  void need(size_t n) {
    HOS_REQUIRE(n <= b.size() && pos <= b.size() - n, HOS_E_FORMAT,
                "unexpected end of GGUF file at byte " + std::to_string(pos));
  }
  template <class T>
  T get() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, b.data() + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    need(n);
    std::string s((const char*)b.data() + pos, (size_t)n);
    pos += n;
    return s;
  }
  // One metadata value of GGUF type vt (src/gguf.rs:196-223); arrays are skipped over (their elements
  // are not needed for the config).
  MetaVal value(uint32_t vt, int depth = 0) {
    HOS_REQUIRE(depth < 4, HOS_E_FORMAT, "GGUF metadata arrays nested too deeply");
    MetaVal v;
    v.type = vt;
    switch (vt) {
      case 0: v.u = get<uint8_t>(); v.is_int = true; break;
      case 1: v.i = get<int8_t>(); v.u = (uint64_t)v.i; v.is_int = true; break;
      case 2: v.u = get<uint16_t>(); v.is_int = true; break;
      case 3: v.i = get<int16_t>(); v.u = (uint64_t)v.i; v.is_int = true; break;
      case 4: v.u = get<uint32_t>(); v.is_int = true; break;
      case 5: v.i = get<int32_t>(); v.u = (uint64_t)v.i; v.is_int = true; break;
      case 6: v.f = get<float>(); v.is_float = true; break;
      case 7: v.u = get<uint8_t>() != 0; break;
      case 8: v.s = str(); v.is_str = true; break;
      case 9: {
        const uint32_t et = get<uint32_t>();
        const uint64_t n = get<uint64_t>();
        for (uint64_t k = 0; k < n; k++) (void)value(et, depth + 1);
        break;
      }
      case 10: v.u = get<uint64_t>(); v.is_int = true; break;
      case 11: v.i = get<int64_t>(); v.u = (uint64_t)v.i; v.is_int = true; break;
      case 12: v.f = get<double>(); v.is_float = true; break;
      default: throw Error(HOS_E_FORMAT, "unknown GGUF value type " + std::to_string(vt));
    }
    if (v.is_int && (vt == 0 || vt == 2 || vt == 4 || vt == 10)) v.i = (int64_t)v.u;
    return v;
  }
};

void read_gguf(const char* path, GgufFile& g) {
  HOS_REQUIRE(path != nullptr, HOS_E_INVALID, "null path");
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  HOS_REQUIRE(f.good(), HOS_E_IO, std::string("cannot open '") + path + "'");
  const std::streamsize n = f.tellg();
  f.seekg(0);
  g.buf.resize((size_t)n);
  HOS_REQUIRE(f.read((char*)g.buf.data(), n).good() || n == 0, HOS_E_IO, std::string("cannot read '") + path + "'");
  Reader r{g.buf};
  const uint32_t magic = r.get<uint32_t>();
  HOS_REQUIRE(std::memcmp(&magic, "GGUF", 4) == 0, HOS_E_FORMAT, "not a GGUF file (bad magic)");
  const uint32_t version = r.get<uint32_t>();
  HOS_REQUIRE(version == 2 || version == 3, HOS_E_FORMAT, "unsupported GGUF version " + std::to_string(version));
  const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
  for (uint64_t k = 0; k < n_kv; k++) {
    std::string key = r.str();
    const uint32_t vt = r.get<uint32_t>();
    g.meta[key] = r.value(vt);
  }
  for (uint64_t k = 0; k < n_tensors; k++) {
    std::string name = r.str();
    TInfo t;
    const uint32_t nd = r.get<uint32_t>();
    HOS_REQUIRE(nd <= 8, HOS_E_FORMAT, "tensor '" + name + "' has " + std::to_string(nd) + " dims");
    for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.get<uint64_t>());
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    g.tensors[name] = t;
  }
  uint64_t align = 32;
  (void)g.meta_u64("general.alignment", &align);
  HOS_REQUIRE(align > 0 && align <= (1u << 30), HOS_E_FORMAT, "general.alignment is 0 or absurdly large");
  g.data_offset = (size_t)((r.pos + align - 1) / align * align);
}

uint64_t n_elements(const TInfo& t) {
  uint64_t n = 1;
  for (uint64_t d : t.dims) {
    HOS_REQUIRE(d == 0 || n <= UINT64_MAX / d, HOS_E_FORMAT, "tensor element count overflows");
    n *= d;
  }
  return n;
}

// Raw bytes of a tensor (src/gguf.rs:513-533).
const uint8_t* raw(const GgufFile& g, const std::string& name, const TInfo& t, size_t* nbytes) {
  const uint64_t n = n_elements(t);
  // every byte count below is at most 4·n: bound n first so no product can wrap
  HOS_REQUIRE(n <= (1ull << 48), HOS_E_FORMAT, "tensor '" + name + "' is larger than any file could hold");
  size_t nb = 0;
  switch (t.type) {
    case T_F32: nb = n * 4; break;
    case T_F16:
    case T_BF16: nb = n * 2; break;
    default: nb = gguf_bytes_for(t.type, n); break;
  }
  HOS_REQUIRE(nb > 0 || n == 0, HOS_E_UNSUPPORTED_QUANT,
              "tensor '" + name + "' has GGUF type " + std::to_string(t.type) +
                  " (supported: F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)");
  HOS_REQUIRE(t.offset <= g.buf.size(), HOS_E_FORMAT, "tensor '" + name + "' data out of bounds");
  const uint64_t start = (uint64_t)g.data_offset + t.offset;
  HOS_REQUIRE(start <= g.buf.size() && nb <= g.buf.size() - start, HOS_E_FORMAT,
              "tensor '" + name + "' data out of bounds");
  *nbytes = nb;
  return g.buf.data() + start;
}

// Every tensor's data must lie inside the file: checked once at open for every type whose size is known
// (raw() checks again before a tensor is read), so a crafted header is a format error up front.
void validate_extents(const GgufFile& g) {
  for (const auto& kv : g.tensors) {
    size_t nb = 0;
    const TInfo& t = kv.second;
    if (t.type == T_F32 || t.type == T_F16 || t.type == T_BF16 || gguf_bytes_for(t.type, 1 << 8) > 0)
      (void)raw(g, kv.first, t, &nb);
  }
}

float half_to_f32(uint16_t h) {
  _Float16 v;
  std::memcpy(&v, &h, 2);
  return (float)v;
}

// The model configuration from the metadata (src/model.rs:721-771, 889-907).
hos_peft_cfg map_config(const GgufFile& g, const hos_peft_cfg* train) {
  const std::string arch = g.meta_str("general.architecture", "llama");
  if (g.has("blk.0.ssm_a")) throw Error(HOS_E_UNSUPPORTED_ARCH, "hybrid SSM models are not trainable here");
  // Arch::detect (src/model.rs:27-42): qwen2moe is the Qwen2 family (shared experts, if any, are not read)
  HOS_REQUIRE(arch == "llama" || arch == "qwen2" || arch == "qwen2moe" || arch == "mistral" || arch == "olmoe",
              HOS_E_UNSUPPORTED_ARCH,
              "architecture '" + arch + "' is not supported by the training step (llama, qwen2, qwen2moe, mistral, olmoe)");
  auto need = [&](const std::string& key) {
    uint64_t v = 0;
    HOS_REQUIRE(g.meta_u64(arch + "." + key, &v), HOS_E_MISSING_META, "missing metadata '" + arch + "." + key + "'");
    return v;
  };
  hos_peft_cfg c{};
  if (train) c = *train;
  c.dim = (int)need("embedding_length");
  c.n_layers = (int)need("block_count");
  c.n_heads = (int)need("attention.head_count");
  uint64_t v = 0;
  c.n_kv_heads = g.meta_u64(arch + ".attention.head_count_kv", &v) ? (int)v : c.n_heads;
  c.ffn_dim = (int)need("feed_forward_length");
  float fv = 0;
  c.rms_eps = g.meta_f32(arch + ".attention.layer_norm_rms_epsilon", &fv) ? fv : 1e-5f;
  c.rope_base = g.meta_f32(arch + ".rope.freq_base", &fv) ? fv : 10000.0f;
  if (g.meta_u64(arch + ".attention.key_length", &v) || g.meta_u64(arch + ".rope.dimension_count", &v))
    c.head_dim = (int)v;
  else
    c.head_dim = c.n_heads > 0 ? c.dim / c.n_heads : 0;
  auto it = g.tensors.find("token_embd.weight");
  HOS_REQUIRE(it != g.tensors.end(), HOS_E_MISSING_TENSOR, "missing tensor 'token_embd.weight'");
  HOS_REQUIRE(c.dim > 0, HOS_E_FORMAT, "embedding_length is 0");
  c.vocab = (int)(n_elements(it->second) / (uint64_t)c.dim);
  c.attn_bias = g.has("blk.0.attn_q.bias") ? 1 : 0;
  c.rope_neox = (arch == "qwen2" || arch == "qwen2moe" || arch == "olmoe") ? 1 : 0;  // Arch::rope_neox, src/model.rs:80-82
  // mixture of experts (src/model.rs:792-795): expert_count > 0 and the stacked expert tensors present
  uint64_t ne = 0, nu = 0;
  (void)g.meta_u64(arch + ".expert_count", &ne);
  (void)g.meta_u64(arch + ".expert_used_count", &nu);
  const bool moe = ne > 0 && g.has("blk.0.ffn_gate_exps.weight");
  c.n_experts = moe ? (int)ne : 0;
  c.n_experts_used = moe ? (int)nu : 0;
  c.qk_norm = g.has("blk.0.attn_q_norm.weight") ? 1 : 0;
  return c;
}

}  // namespace

extern "C" {

int hos_gguf_config(const char* path, hos_peft_cfg* out, char* err, size_t err_len) {
  try {
    HOS_REQUIRE(out != nullptr, HOS_E_INVALID, "null output");
    GgufFile g;
    read_gguf(path, g);
    validate_extents(g);
    *out = map_config(g, out);
    return HOS_OK;
  } catch (const Error& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    return e.code;
  } catch (const std::exception& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    return HOS_E_IO;
  }
}

int hos_peft_create_from_gguf(hos_ctx* ctx, const char* path, const hos_peft_cfg* train, hos_peft** out,
                              hos_peft_cfg* out_cfg) {
  if (!ctx || !out) return HOS_E_INVALID;
  *out = nullptr;
  GgufFile g;
  hos_peft_cfg c{};
  try {
    read_gguf(path, g);
    validate_extents(g);
    c = map_config(g, train);
  } catch (const Error& e) {
    std::fprintf(stderr, "hos_peft_create_from_gguf: %s\n", e.what());
    return e.code;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "hos_peft_create_from_gguf: %s\n", e.what());
    return HOS_E_IO;
  }
  if (out_cfg) *out_cfg = c;
  hos_peft* p = nullptr;
  int rc = hos_peft_create(ctx, &c, &p);
  if (rc) return rc;
  std::vector<float> widened;
  for (const auto& kv : g.tensors) {
    const std::string& name = kv.first;
    const TInfo& t = kv.second;
    const bool wanted = name == "token_embd.weight" || name == "output.weight" || name == "output_norm.weight" ||
                        name.rfind("blk.", 0) == 0;
    if (!wanted) continue;
    size_t nb = 0;
    const uint8_t* bytes = nullptr;
    try {
      bytes = raw(g, name, t, &nb);
    } catch (const Error& e) {
      std::fprintf(stderr, "hos_peft_create_from_gguf: %s\n", e.what());
      hos_peft_destroy(p);
      return e.code;
    }
    const size_t cols = t.dims.empty() ? 1 : (size_t)t.dims[0];
    const size_t rows = t.dims.size() > 1 ? (size_t)(n_elements(t) / (t.dims[0] ? t.dims[0] : 1)) : 1;
    uint32_t type = t.type;
    const bool router = name.size() > 19 && name.compare(name.size() - 19, 19, "ffn_gate_inp.weight") == 0;
    if ((t.type == T_F16 || t.type == T_BF16) && (t.dims.size() == 1 || router)) {  // norms, biases, router: F32
      const size_t n = nb / 2;
      widened.resize(n);
      for (size_t k = 0; k < n; k++) {
        uint16_t h;
        std::memcpy(&h, bytes + 2 * k, 2);
        if (t.type == T_F16) {
          widened[k] = half_to_f32(h);
        } else {
          const uint32_t u = (uint32_t)h << 16;
          std::memcpy(&widened[k], &u, 4);
        }
      }
      bytes = (const uint8_t*)widened.data();
      nb = n * 4;
      type = T_F32;
    }
    rc = hos_peft_set_tensor(p, name.c_str(), bytes, nb, type, rows, cols);
    if (rc) {
      std::fprintf(stderr, "hos_peft_create_from_gguf: %s\n", hos_peft_last_error(p));
      hos_peft_destroy(p);
      return rc;
    }
  }
  *out = p;
  return HOS_OK;
}

}  // extern "C"
