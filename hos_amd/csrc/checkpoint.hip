// Adapter / optimizer checkpoints in the .hos capsule layout (host code).
//
// Layout (src/format.rs:1-26, writer :287-346, reader :401-485), little-endian:
//   "HOSF" | version u32 (2) | flags u32 (0) | card_len u32 | card JSON | n_tensors u32
//   per tensor: name_len u32, name, role u8, dtype u8 (v2+), ndim u32, dims u32[ndim], n_floats u64,
//               n_bytes u64 (v2+), checksum u64 (FNV-1a 64 of the stored bytes)
//   zero pad to 32 | each tensor's stored bytes, zero padded to 32 | file checksum u64 (FNV-1a 64 of all
//   bytes before it)
// Tensors written here (role, dtype F32):
//   lora.{l}.a{t}, lora.{l}.b{t}  ROLE_WEIGHT, A [in, r], B [r, out]; per layer, per adapted target in the
//                                 order q,k,v,o,gate,up,down, A before B (PeftModel::adapter_tensors and
//                                 params_bank, src/peft.rs:294-300, 731-740: lora.{i}.{aq,bq,av,bv})
//   opt.m.{k}, opt.v.{k}          ROLE_OPT_STATE, [n], AdamW moments of the k-th parameter in that order
//   opt.step, opt.lr, opt.beta1, opt.beta2, opt.wd   ROLE_SCALAR, [1]   (src/main.rs:6276-6307)
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

#include "ctx.hpp"
#include "peft_internal.hpp"

using namespace hos;

namespace {

constexpr uint8_t ROLE_WEIGHT = 0, ROLE_OPT_STATE = 4, ROLE_SCALAR = 5;  // src/format.rs:117-122
constexpr uint8_t DTYPE_F32 = 0;                                          // src/format.rs:125
const char* const TARGET_NAME[7] = {"q", "k", "v", "o", "gate", "up", "down"};

uint64_t fnv1a64(const uint8_t* b, size_t n, uint64_t h = 0xcbf29ce484222325ull) {
  for (size_t i = 0; i < n; i++) {
    h ^= b[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

struct Tensor {
  std::string name;
  uint8_t role = ROLE_WEIGHT, dtype = DTYPE_F32;
  std::vector<uint32_t> shape;
  uint64_t nfloats = 0;
  std::vector<float> data;            // written tensors
  const uint8_t* stored = nullptr;    // read tensors: bytes inside the file buffer
  uint64_t nbytes = 0, checksum = 0;
};

// The adapter tensors of the model in checkpoint order (data read back from the device arena).
void adapter_tensors(hos_peft* p, const PeftShape& s, PeftBuf which, const char* prefix, std::vector<Tensor>& out,
                     bool flat) {
  int k = 0;
  if (s.rga) {  // named tensors; the optimizer state follows the parameter order
    for (auto& [name, shape] : peft_rga_tensors(p, flat)) {
      Tensor t;
      t.data.resize((size_t)shape[0] * shape[1]);
      peft_rga_io(p, which, name, t.data.data(), t.data.size(), false);
      t.nfloats = t.data.size();
      t.role = flat ? ROLE_OPT_STATE : ROLE_WEIGHT;
      t.name = flat ? std::string(prefix) + std::to_string(k++) : name;
      t.shape = flat ? std::vector<uint32_t>{(uint32_t)t.nfloats} : shape;
      out.push_back(std::move(t));
    }
    return;
  }
  for (int l = 0; l < s.L; l++)
    for (int t = 0; t < 7; t++) {
      if (!((s.targets >> t) & 1u)) continue;
      Tensor a, b;
      a.data.resize((size_t)s.in[t] * s.r);
      b.data.resize((size_t)s.r * s.out[t]);
      peft_factor_io(p, which, l, t, a.data.data(), b.data.data(), false);
      for (Tensor* x : {&a, &b}) {
        x->role = flat ? ROLE_OPT_STATE : ROLE_WEIGHT;
        x->nfloats = x->data.size();
      }
      if (flat) {
        a.name = std::string(prefix) + std::to_string(k++);
        b.name = std::string(prefix) + std::to_string(k++);
        a.shape = {(uint32_t)a.nfloats};
        b.shape = {(uint32_t)b.nfloats};
      } else {
        a.name = "lora." + std::to_string(l) + ".a" + TARGET_NAME[t];
        b.name = "lora." + std::to_string(l) + ".b" + TARGET_NAME[t];
        a.shape = {(uint32_t)s.in[t], (uint32_t)s.r};
        b.shape = {(uint32_t)s.r, (uint32_t)s.out[t]};
      }
      out.push_back(std::move(a));
      out.push_back(std::move(b));
    }
}

// model_id (src/format.rs:100-111): FNV-1a 64 over every tensor's f32 little-endian bytes, as 16 hex digits.
std::string model_id(const std::vector<Tensor>& ts) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (const Tensor& t : ts) h = fnv1a64((const uint8_t*)t.data.data(), t.data.size() * 4, h);
  char buf[17];
  std::snprintf(buf, sizeof(buf), "%016llx", (unsigned long long)h);
  return buf;
}

Tensor scalar(const char* name, float v) {
  Tensor t;
  t.name = name;
  t.role = ROLE_SCALAR;
  t.shape = {1};
  t.nfloats = 1;
  t.data = {v};
  return t;
}

template <class T>
void put(std::vector<uint8_t>& b, T v) {
  const size_t n = b.size();
  b.resize(n + sizeof(T));
  std::memcpy(b.data() + n, &v, sizeof(T));
}
void pad32(std::vector<uint8_t>& b) { b.resize((b.size() + 31) / 32 * 32, 0); }

void write_capsule(const char* path, const std::string& card, const std::vector<Tensor>& ts) {
  std::vector<uint8_t> b;
  b.insert(b.end(), {'H', 'O', 'S', 'F'});
  put<uint32_t>(b, 2);
  put<uint32_t>(b, 0);
  put<uint32_t>(b, (uint32_t)card.size());
  b.insert(b.end(), card.begin(), card.end());
  put<uint32_t>(b, (uint32_t)ts.size());
  for (const Tensor& t : ts) {
    put<uint32_t>(b, (uint32_t)t.name.size());
    b.insert(b.end(), t.name.begin(), t.name.end());
    put<uint8_t>(b, t.role);
    put<uint8_t>(b, DTYPE_F32);
    put<uint32_t>(b, (uint32_t)t.shape.size());
    for (uint32_t d : t.shape) put<uint32_t>(b, d);
    put<uint64_t>(b, t.data.size());
    put<uint64_t>(b, t.data.size() * 4);
    put<uint64_t>(b, fnv1a64((const uint8_t*)t.data.data(), t.data.size() * 4));
  }
  pad32(b);
  for (const Tensor& t : ts) {
    const uint8_t* d = (const uint8_t*)t.data.data();
    b.insert(b.end(), d, d + t.data.size() * 4);
    pad32(b);
  }
  put<uint64_t>(b, fnv1a64(b.data(), b.size()));
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  HOS_REQUIRE(f.good(), HOS_E_IO, std::string("cannot create '") + path + "'");
  f.write((const char*)b.data(), (std::streamsize)b.size());
  f.close();
  HOS_REQUIRE(f.good(), HOS_E_IO, std::string("cannot write '") + path + "'");
}

struct Capsule {
  std::vector<uint8_t> buf;
  uint32_t version = 0;
  std::string card;
  std::vector<Tensor> tensors;
  std::map<std::string, size_t> index;
};

struct Cursor {
  const std::vector<uint8_t>& b;
  size_t p = 0;
  const uint8_t* take(uint64_t n) {
    HOS_REQUIRE(n <= b.size() && p <= b.size() - n, HOS_E_FORMAT, "truncated .hos file at byte " + std::to_string(p));
    const uint8_t* r = b.data() + p;
    p += n;
    return r;
  }
  template <class T>
  T get() {
    T v;
    std::memcpy(&v, take(sizeof(T)), sizeof(T));
    return v;
  }
  void align32() { p = std::min(b.size(), (p + 31) / 32 * 32); }
};

void read_file(const char* path, std::vector<uint8_t>& buf) {
  HOS_REQUIRE(path != nullptr, HOS_E_INVALID, "null path");
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  HOS_REQUIRE(f.good(), HOS_E_IO, std::string("cannot open '") + path + "'");
  const std::streamsize n = f.tellg();
  f.seekg(0);
  buf.resize((size_t)n);
  if (n > 0) HOS_REQUIRE(f.read((char*)buf.data(), n).good(), HOS_E_IO, std::string("cannot read '") + path + "'");
}

// load_raw (src/format.rs:401-485): header, card, tensor table (v1: no dtype / byte count), 32-byte
// aligned data, per-tensor checksum verified.
void read_capsule(const char* path, Capsule& c, bool header_only = false) {
  read_file(path, c.buf);
  Cursor r{c.buf};
  HOS_REQUIRE(c.buf.size() >= 4 && std::memcmp(r.take(4), "HOSF", 4) == 0, HOS_E_FORMAT, "not a HOS file");
  c.version = r.get<uint32_t>();
  (void)r.get<uint32_t>();  // flags
  const uint32_t card_len = r.get<uint32_t>();
  const uint8_t* cb = r.take(card_len);
  c.card.assign((const char*)cb, card_len);
  if (header_only) return;
  const uint32_t n = r.get<uint32_t>();
  for (uint32_t i = 0; i < n; i++) {
    Tensor t;
    const uint32_t nl = r.get<uint32_t>();
    t.name.assign((const char*)r.take(nl), nl);
    t.role = r.get<uint8_t>();
    t.dtype = c.version >= 2 ? r.get<uint8_t>() : DTYPE_F32;
    const uint32_t nd = r.get<uint32_t>();
    HOS_REQUIRE(nd <= 16, HOS_E_FORMAT, "tensor '" + t.name + "' has " + std::to_string(nd) + " dims");
    for (uint32_t d = 0; d < nd; d++) t.shape.push_back(r.get<uint32_t>());
    t.nfloats = r.get<uint64_t>();
    HOS_REQUIRE(t.nfloats <= c.buf.size(), HOS_E_FORMAT, "tensor '" + t.name + "' element count exceeds the file");
    t.nbytes = c.version >= 2 ? r.get<uint64_t>() : t.nfloats * 4;
    t.checksum = r.get<uint64_t>();
    c.tensors.push_back(std::move(t));
  }
  r.align32();
  for (Tensor& t : c.tensors) {
    t.stored = r.take(t.nbytes);
    r.align32();
    HOS_REQUIRE(fnv1a64(t.stored, t.nbytes) == t.checksum, HOS_E_FORMAT, "checksum mismatch in tensor " + t.name);
  }
  for (size_t i = 0; i < c.tensors.size(); i++) c.index[c.tensors[i].name] = i;
}

// One tensor's f32 values; F32 is the only stored encoding adapters and optimizer state use
// (src/format.rs:171-174 keeps optimizer state and scalars full precision).
void decode_f32(const Tensor& t, std::vector<float>& out) {
  HOS_REQUIRE(t.dtype == DTYPE_F32, HOS_E_UNSUPPORTED_QUANT,
              "tensor '" + t.name + "' is stored with dtype " + std::to_string(t.dtype) + " (F32 expected)");
  HOS_REQUIRE(t.nbytes == t.nfloats * 4, HOS_E_FORMAT, "tensor '" + t.name + "' byte count mismatch");
  out.resize(t.nfloats);
  if (t.nbytes) std::memcpy(out.data(), t.stored, t.nbytes);
}

const Tensor& need(const Capsule& c, const std::string& name) {
  auto it = c.index.find(name);
  HOS_REQUIRE(it != c.index.end(), HOS_E_MISSING_TENSOR, "missing tensor '" + name + "'");
  return c.tensors[it->second];
}

void need_shape(const Tensor& t, std::vector<uint32_t> want) {
  uint64_t n = 1;
  for (uint32_t d : want) n *= d;
  HOS_REQUIRE(t.shape == want && t.nfloats == n, HOS_E_FORMAT,
              "tensor '" + t.name + "' has the wrong shape for this model");
}

std::string default_card(const PeftShape& s, const std::string& id) {
  // Card::new + the adapter fields of save_adapter (src/format.rs:79-97, src/main.rs:2646-2676); keys in
  // serde's order, the arch object's keys sorted as serde_json's map keeps them.
  char buf[640];
  const char* method = s.rga ? "rga" : "lora";
  std::snprintf(buf, sizeof(buf),
                "{\"format\":\"hos\",\"spec\":1,\"name\":\"hos-peft-%s\",\"id\":\"%s\",\"mode\":\"adapter\","
                "\"arch\":{\"block_count\":%d,\"method\":\"%s\",\"source_format\":\"hos-peft\"},"
                "\"provenance\":{\"created\":\"\",\"engine\":\"hos-peft\",\"dataset\":\"\",\"dataset_hash\":\"\"},"
                "\"resume\":{\"seed\":0,\"step\":%llu,\"rng_state\":0},\"history\":[],\"lineage\":[]}",
                method, id.c_str(), s.L, method, (unsigned long long)s.step);
  return buf;
}

int copy_out(const std::string& s, char* out, size_t len, size_t* needed) {
  if (needed) *needed = s.size() + 1;
  if (out && len) {
    const size_t n = std::min(len - 1, s.size());
    std::memcpy(out, s.data(), n);
    out[n] = 0;
  }
  return HOS_OK;
}

}  // namespace

extern "C" {

int hos_peft_adapter_id(hos_peft* p, char* out17) {
  if (!p || !out17) return HOS_E_INVALID;
  return peft_call(p, [&] {
    std::vector<Tensor> ts;
    adapter_tensors(p, peft_shape(p), PEFT_PARAM, "", ts, false);
    std::snprintf(out17, 17, "%s", model_id(ts).c_str());
  });
}

int hos_peft_base_id(hos_peft* p, char* out17) {
  if (!p || !out17) return HOS_E_INVALID;
  return peft_call(p, [&] {
    std::vector<float> e;
    peft_token_embedding(p, e);
    std::snprintf(out17, 17, "%016llx", (unsigned long long)fnv1a64((const uint8_t*)e.data(), e.size() * 4));
  });
}

int hos_peft_save_hos(hos_peft* p, const char* path, const char* card_json, int with_optimizer) {
  if (!p || !path) return HOS_E_INVALID;
  return peft_call(p, [&] {
    const PeftShape s = peft_shape(p);
    std::vector<Tensor> ts;
    adapter_tensors(p, s, PEFT_PARAM, "", ts, false);
    const std::string card = card_json ? std::string(card_json) : default_card(s, model_id(ts));
    if (with_optimizer) {
      std::vector<Tensor> m, v;
      adapter_tensors(p, s, PEFT_ADAM_M, "opt.m.", m, true);
      adapter_tensors(p, s, PEFT_ADAM_V, "opt.v.", v, true);
      for (size_t k = 0; k < m.size(); k++) {  // opt.m.k, opt.v.k interleaved (src/main.rs:6276-6289)
        ts.push_back(std::move(m[k]));
        ts.push_back(std::move(v[k]));
      }
      ts.push_back(scalar("opt.step", (float)s.step));
      ts.push_back(scalar("opt.lr", s.lr));
      ts.push_back(scalar("opt.beta1", 0.9f));
      ts.push_back(scalar("opt.beta2", 0.95f));
      ts.push_back(scalar("opt.wd", s.wd));
    }
    write_capsule(path, card, ts);
  });
}

int hos_peft_load_hos(hos_peft* p, const char* path, int with_optimizer) {
  if (!p || !path) return HOS_E_INVALID;
  return peft_call(p, [&] {
    Capsule c;
    read_capsule(path, c);
    const PeftShape s = peft_shape(p);
    // Validate and decode everything before touching the device, so a bad file leaves the model as it was.
    struct Pair {
      int l, t;
      std::vector<float> a, b, ma, mb, va, vb;
    };
    std::vector<Pair> pairs;
    // RGA: every adapter tensor by name (+ its moments by parameter index)
    struct Named {
      std::string name;
      std::vector<float> v, m, vv;
    };
    std::vector<Named> rn;
    if (s.rga) {
      for (auto& [name, shape] : peft_rga_tensors(p, false)) {
        Named q{name};
        const Tensor& t = need(c, name);
        need_shape(t, shape);
        decode_f32(t, q.v);
        rn.push_back(std::move(q));
      }
      if (with_optimizer) {
        int kk = 0;
        for (auto& [name, shape] : peft_rga_tensors(p, true)) {
          Named* q = nullptr;
          for (auto& x : rn)
            if (x.name == name) q = &x;
          const uint32_t n = shape[0] * shape[1];
          const Tensor& tm = need(c, "opt.m." + std::to_string(kk));
          const Tensor& tv = need(c, "opt.v." + std::to_string(kk));
          need_shape(tm, {n});
          need_shape(tv, {n});
          decode_f32(tm, q->m);
          decode_f32(tv, q->vv);
          kk++;
        }
      }
    }
    int k = 0;
    for (int l = 0; l < (s.rga ? 0 : s.L); l++)
      for (int t = 0; t < 7; t++) {
        if (!((s.targets >> t) & 1u)) continue;
        Pair q{l, t};
        const std::string pre = "lora." + std::to_string(l) + ".";
        const Tensor& ta = need(c, pre + "a" + TARGET_NAME[t]);
        const Tensor& tb = need(c, pre + "b" + TARGET_NAME[t]);
        need_shape(ta, {(uint32_t)s.in[t], (uint32_t)s.r});
        need_shape(tb, {(uint32_t)s.r, (uint32_t)s.out[t]});
        decode_f32(ta, q.a);
        decode_f32(tb, q.b);
        if (with_optimizer) {
          const Tensor* mv[4] = {&need(c, "opt.m." + std::to_string(k)), &need(c, "opt.m." + std::to_string(k + 1)),
                                 &need(c, "opt.v." + std::to_string(k)), &need(c, "opt.v." + std::to_string(k + 1))};
          need_shape(*mv[0], {(uint32_t)q.a.size()});
          need_shape(*mv[1], {(uint32_t)q.b.size()});
          need_shape(*mv[2], {(uint32_t)q.a.size()});
          need_shape(*mv[3], {(uint32_t)q.b.size()});
          decode_f32(*mv[0], q.ma);
          decode_f32(*mv[1], q.mb);
          decode_f32(*mv[2], q.va);
          decode_f32(*mv[3], q.vb);
        }
        k += 2;
        pairs.push_back(std::move(q));
      }
    float step = 0, lr = s.lr, wd = s.wd;
    if (with_optimizer) {
      std::vector<float> v;
      const char* names[3] = {"opt.step", "opt.lr", "opt.wd"};
      float* dst[3] = {&step, &lr, &wd};
      for (int i = 0; i < 3; i++) {
        const Tensor& t = need(c, names[i]);
        decode_f32(t, v);
        HOS_REQUIRE(v.size() == 1, HOS_E_FORMAT, std::string("'") + names[i] + "' is not a scalar");
        *dst[i] = v[0];
      }
      HOS_REQUIRE(step >= 0 && step <= 2147483647.0f && step == (float)(uint64_t)step, HOS_E_FORMAT,
                  "opt.step is not a step count");
    }
    for (Named& q : rn) {
      peft_rga_io(p, PEFT_PARAM, q.name, q.v.data(), q.v.size(), true);
      if (with_optimizer) {
        peft_rga_io(p, PEFT_ADAM_M, q.name, q.m.data(), q.m.size(), true);
        peft_rga_io(p, PEFT_ADAM_V, q.name, q.vv.data(), q.vv.size(), true);
      }
    }
    for (Pair& q : pairs) {
      peft_factor_io(p, PEFT_PARAM, q.l, q.t, q.a.data(), q.b.data(), true);
      if (with_optimizer) {
        peft_factor_io(p, PEFT_ADAM_M, q.l, q.t, q.ma.data(), q.mb.data(), true);
        peft_factor_io(p, PEFT_ADAM_V, q.l, q.t, q.va.data(), q.vb.data(), true);
      }
    }
    if (with_optimizer) peft_set_adam_state(p, (uint64_t)step, lr, wd);
  });
}

int hos_format_verify(const char* path, size_t* n_tensors, char* err, size_t err_len) {
  try {
    Capsule c;
    read_capsule(path, c);
    std::vector<float> v;
    for (const Tensor& t : c.tensors)
      if (t.dtype == DTYPE_F32) decode_f32(t, v);
    if (n_tensors) *n_tensors = c.tensors.size();
    return HOS_OK;
  } catch (const Error& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    return e.code;
  } catch (const std::exception& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    return HOS_E_IO;
  }
}

int hos_format_card(const char* path, char* out, size_t len, size_t* needed) {
  try {
    Capsule c;
    read_capsule(path, c, true);
    return copy_out(c.card, out, len, needed);
  } catch (const Error& e) {
    if (out && len) std::snprintf(out, len, "%s", e.what());
    return e.code;
  } catch (const std::exception& e) {
    if (out && len) std::snprintf(out, len, "%s", e.what());
    return HOS_E_IO;
  }
}

}  // extern "C"
