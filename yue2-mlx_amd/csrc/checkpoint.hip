// Checkpoint directory loader: the drop-in for ARModel(directory, precision,
// verify = false) (native/src/ar.cpp:133-238). Host code only.
//
//   conversion.json  schema-1 manifest; precisions[precision] names the AR
//                    file "ar-<precision>.safetensors" (bf16: dtype
//                    "bfloat16"; 8bit/4bit: affine, group 64, linear only)
//   config.json      architecture; the reference's checks (ar.cpp:161-192),
//                    with the YuE2 dimensions required when `strict`
//   ar-*.safetensors 8-byte little-endian header length, JSON header
//                    {name: {dtype, shape, data_offsets}}, then the data
//
// Every tensor the reference requires must be present with its shape and
// dtype and nothing else (ar.cpp:193-236, same messages). The file is mapped
// read-only and its tensors are handed to yuear_engine_create, which copies
// them to the device. With the affine-quantized precisions every linear (the
// seven projections of each layer and the lm_head) is U32 codes
// [rows][k * bits / 32] plus BF16 scales and biases [rows][k / 64]
// (ar.cpp:209-214); the embedding and the norms stay BF16.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/yuear.h"
#include "abi_util.h"
#include "json.h"

namespace yuear {
namespace {

constexpr int kVocabYuE2 = 184704, kContextYuE2 = 24576;  // types.hpp:18-19

std::string read_text(const std::string &path, size_t max_bytes) {
  struct stat st;
  if (::stat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode))
    throw Error("FileNotFoundError", path);
  if (size_t(st.st_size) > max_bytes)
    invalid(path + " is too large");
  std::ifstream f(path, std::ios::binary);
  if (!f)
    throw Error("FileNotFoundError", path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

json::Value read_json(const std::string &path) {
  const std::string text = read_text(path, size_t(16) << 20);
  try {
    return json::parse(text);
  } catch (const std::exception &e) {
    invalid(path + ": " + e.what());
  }
}

const json::Value *field(const json::Value &o, const char *k) { return o.get(k); }

bool is_int(const json::Value *v) { return v && v->is_number() && v->integer; }

// manifest (ar.cpp:137-160)
std::string check_manifest(const json::Value &m, const std::string &precision) {
  const json::Value *schema = field(m, "schema");
  if (!m.is_object() || !is_int(schema) || schema->inum != 1)
    invalid("conversion.json must be a schema-1 manifest");
  const json::Value *prec = field(m, "precisions");
  const json::Value *entry = prec && prec->is_object() ? prec->get(precision) : nullptr;
  if (!entry || !entry->is_object())
    throw Error("FileNotFoundError",
                "Converted artifact does not contain " + precision + " AR weights");
  const std::string filename = "ar-" + precision + ".safetensors";
  const json::Value *ar = field(*entry, "ar");
  if (!ar || !ar->is_string() || ar->str != filename)
    invalid("Manifest AR filename does not match precision");
  if (precision == "bf16") {
    const json::Value *dt = field(*entry, "dtype");
    if (!dt || !dt->is_string() || dt->str != "bfloat16")
      invalid("BF16 manifest entry must declare dtype='bfloat16'");
  } else {
    const int bits = precision == "8bit" ? 8 : 4;
    const json::Value *b = field(*entry, "bits"), *g = field(*entry, "group_size"),
                      *mode = field(*entry, "mode"), *lin = field(*entry, "linear_only");
    if (!is_int(b) || b->inum != bits || !is_int(g) || g->inum != 64 || !mode ||
        !mode->is_string() || mode->str != "affine" || !lin || lin->kind != json::Value::Bool ||
        !lin->b)
      invalid("Invalid affine quantization settings in AR manifest");
  }
  return filename;
}

// config.json (ar.cpp:161-192); strict: the YuE2 generator dimensions
yuear_model_config check_config(const json::Value &c, bool strict) {
  if (!c.is_object())
    invalid("config.json must contain a JSON object");
  struct Want {
    const char *key;
    long long yue2;
  };
  const Want ints[] = {{"hidden_size", 2048},       {"intermediate_size", 6144},
                       {"num_hidden_layers", 28},   {"num_attention_heads", 16},
                       {"num_key_value_heads", 8},  {"head_dim", 128},
                       {"vocab_size", kVocabYuE2},  {"max_position_embeddings", kContextYuE2}};
  long long got[8];
  for (int i = 0; i < 8; ++i) {
    const json::Value *v = field(c, ints[i].key);
    json::Value dflt;
    if (!v && std::string(ints[i].key) == "max_position_embeddings") {
      dflt.kind = json::Value::Number;
      dflt.integer = true;
      dflt.inum = kContextYuE2;
      dflt.num = kContextYuE2;
      v = &dflt;
    }
    if (strict && !(v && v->is_number() && v->num == double(ints[i].yue2)))
      invalid(std::string("Incompatible YuE2 config: ") + ints[i].key);
    if (!is_int(v) || v->inum < 1 || v->inum > (1LL << 30))
      invalid(std::string("Generator config field ") + ints[i].key +
              " must be a positive integer");
    got[i] = v->inum;
  }
  const json::Value *theta = field(c, "rope_theta");
  if (strict && !(theta && theta->is_number() && theta->num == 1000000.0))
    invalid("Incompatible YuE2 config: rope_theta");
  if (!theta || !theta->is_number() || !std::isfinite(theta->num) || theta->num <= 0)
    invalid("Incompatible YuE2 config: rope_theta");
  const json::Value *tie = field(c, "tie_word_embeddings");
  if (tie && !(tie->kind == json::Value::Bool && !tie->b))
    invalid("YuE2 requires untied input and output embeddings");
  const json::Value *scaling = field(c, "rope_scaling");
  if (scaling && scaling->kind != json::Value::Null &&
      !(scaling->is_object() && scaling->obj.empty()))
    invalid("YuE2 uses fixed base RoPE without scaling");
  const json::Value *act = field(c, "hidden_act");
  if (act && !(act->is_string() && act->str == "silu"))
    invalid("Incompatible YuE2 config: hidden_act must be silu");
  const json::Value *eps = field(c, "rms_norm_eps");
  if (!eps || !eps->is_number() || !std::isfinite(eps->num) || eps->num <= 0)
    invalid("rms_norm_eps must be finite and positive");
  yuear_model_config k{};
  k.hidden_size = int32_t(got[0]);
  k.intermediate_size = int32_t(got[1]);
  k.num_hidden_layers = int32_t(got[2]);
  k.num_attention_heads = int32_t(got[3]);
  k.num_key_value_heads = int32_t(got[4]);
  k.head_dim = int32_t(got[5]);
  k.vocab_size = int32_t(got[6]);
  k.max_position_embeddings = int32_t(got[7]);
  k.rms_norm_eps = float(eps->num);
  k.rope_theta = theta->num;
  k.qk_norm = 1;  // the reference graph always applies q_norm / k_norm (ar.cpp:268-275)
  return k;
}

// Read-only mapping of the safetensors file.
struct Mapping {
  void *base = MAP_FAILED;
  size_t bytes = 0;
  ~Mapping() {
    if (base != MAP_FAILED)
      ::munmap(base, bytes);
  }
};

struct Loaded {
  yuear_model_config config{};
  Mapping map;
  std::vector<std::string> names;
  std::vector<yuear_tensor> tensors;
  // tensors whose file offset is not a multiple of their element size
  std::vector<std::vector<uint32_t>> realigned;
};

struct TensorSpec {
  std::vector<long long> shape;
  bool u32;  // U32 codes, else BF16
};

// The expected tensors, shapes and dtypes (ar.cpp:193-233) for a config and
// the quantization bits (0: bf16).
std::map<std::string, TensorSpec> expected_tensors(const yuear_model_config &k, int bits) {
  const long long H = k.hidden_size, F = k.intermediate_size, D = k.head_dim,
                  Q = k.num_attention_heads * D, KV = k.num_key_value_heads * D,
                  V = k.vocab_size;
  std::map<std::string, TensorSpec> e;
  auto norm = [&](const std::string &n, long long width) { e[n + ".weight"] = {{width}, false}; };
  auto linear = [&](const std::string &n, long long out, long long in) {
    if (!bits) {
      e[n + ".weight"] = {{out, in}, false};
      return;
    }
    e[n + ".weight"] = {{out, in * bits / 32}, true};
    e[n + ".scales"] = {{out, in / 64}, false};
    e[n + ".biases"] = {{out, in / 64}, false};
  };
  e["model.embed_tokens.weight"] = {{V, H}, false};
  norm("model.norm", H);
  linear("lm_head", V, H);
  for (int i = 0; i < k.num_hidden_layers; ++i) {
    const std::string n = "model.layers." + std::to_string(i);
    norm(n + ".input_layernorm", H);
    norm(n + ".post_attention_layernorm", H);
    norm(n + ".self_attn.q_norm", D);
    norm(n + ".self_attn.k_norm", D);
    linear(n + ".self_attn.q_proj", Q, H);
    linear(n + ".self_attn.k_proj", KV, H);
    linear(n + ".self_attn.v_proj", KV, H);
    linear(n + ".self_attn.o_proj", H, Q);
    linear(n + ".mlp.gate_proj", F, H);
    linear(n + ".mlp.up_proj", F, H);
    linear(n + ".mlp.down_proj", H, F);
  }
  return e;
}

void open_checkpoint(const std::string &dir, const std::string &precision, bool strict,
                     bool map_data, Loaded &out) {
  if (precision != "bf16" && precision != "8bit" && precision != "4bit")
    invalid("precision must be 'bf16', '8bit', or '4bit'");
  struct stat st;
  if (::stat(dir.c_str(), &st) != 0 || !S_ISDIR(st.st_mode))
    throw Error("FileNotFoundError", dir);
  const std::string filename = check_manifest(read_json(dir + "/conversion.json"), precision);
  out.config = check_config(read_json(dir + "/config.json"), strict);
  const int bits = precision == "bf16" ? 0 : precision == "8bit" ? 8 : 4;

  const std::string path = dir + "/" + filename;
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0)
    throw Error("FileNotFoundError", path);
  struct stat fs;
  if (::fstat(fd, &fs) != 0 || !S_ISREG(fs.st_mode)) {
    ::close(fd);
    throw Error("FileNotFoundError", path);
  }
  const size_t file_bytes = size_t(fs.st_size);
  unsigned char len8[8];
  if (file_bytes < 8 || ::pread(fd, len8, 8, 0) != 8) {
    ::close(fd);
    invalid(filename + ": truncated safetensors header");
  }
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i)
    hlen = (hlen << 8) | len8[i];
  if (hlen > file_bytes - 8 || hlen > (uint64_t(100) << 20)) {
    ::close(fd);
    invalid(filename + ": invalid safetensors header length");
  }
  std::string header(size_t(hlen), '\0');
  if (hlen && ::pread(fd, header.data(), size_t(hlen), 8) != ssize_t(hlen)) {
    ::close(fd);
    invalid(filename + ": truncated safetensors header");
  }
  if (map_data) {
    out.map.bytes = file_bytes;
    out.map.base = ::mmap(nullptr, file_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
  }
  ::close(fd);
  if (map_data && out.map.base == MAP_FAILED)
    throw Error("OSError", "cannot map " + path);
  json::Value h;
  try {
    h = json::parse(header);
  } catch (const std::exception &e) {
    invalid(filename + ": " + e.what());
  }
  if (!h.is_object())
    invalid(filename + ": safetensors header must be a JSON object");
  const size_t data0 = 8 + size_t(hlen), data_bytes = file_bytes - data0;

  const auto expected = expected_tensors(out.config, bits);
  std::set<std::string> seen;
  for (const auto &[name, t] : h.obj) {
    if (name == "__metadata__")
      continue;
    auto it = expected.find(name);
    if (it == expected.end())
      invalid("Unexpected AR tensor: " + name);
    const json::Value *dt = t.get("dtype"), *shape = t.get("shape"), *offs = t.get("data_offsets");
    const TensorSpec &spec = it->second;
    const long long esize = spec.u32 ? 4 : 2;
    bool ok = dt && dt->is_string() && dt->str == (spec.u32 ? "U32" : "BF16") && shape &&
              shape->is_array() && shape->arr.size() == spec.shape.size();
    long long numel = 1;
    for (size_t d = 0; ok && d < shape->arr.size(); ++d) {
      const json::Value &s = shape->arr[d];
      ok = is_int(&s) && s.inum == spec.shape[d];
      numel *= ok ? s.inum : 1;
    }
    if (!ok)
      invalid("Incompatible AR tensor shape/dtype: " + name);
    if (!offs || !offs->is_array() || offs->arr.size() != 2 || !is_int(&offs->arr[0]) ||
        !is_int(&offs->arr[1]) || offs->arr[0].inum < 0 || offs->arr[1].inum < offs->arr[0].inum ||
        uint64_t(offs->arr[1].inum) > data_bytes ||
        offs->arr[1].inum - offs->arr[0].inum != numel * esize)
      invalid(filename + ": invalid data offsets for " + name);
    seen.insert(name);
    if (map_data) {
      const size_t at = data0 + size_t(offs->arr[0].inum);
      const unsigned char *p = static_cast<const unsigned char *>(out.map.base) + at;
      const void *data = p;
      if (at % size_t(esize)) {  // safetensors does not promise alignment
        const size_t bytes = size_t(numel * esize);
        out.realigned.emplace_back((bytes + 3) / 4);
        std::memcpy(out.realigned.back().data(), p, bytes);
        data = out.realigned.back().data();
      }
      out.names.push_back(name);
      out.tensors.push_back(yuear_tensor{nullptr, data, numel,
                                         spec.u32 ? YUEAR_DTYPE_U32 : YUEAR_DTYPE_BF16});
    }
  }
  for (const auto &kv : expected)
    if (!seen.count(kv.first))
      invalid("Missing AR tensor: " + kv.first);
  for (size_t i = 0; i < out.tensors.size(); ++i)
    out.tensors[i].name = out.names[i].c_str();
}

}  // namespace
}  // namespace yuear

using namespace yuear;

extern "C" yuear_status yuear_checkpoint_inspect(const char *directory, const char *precision,
                                                 int32_t strict, yuear_model_config *config_out,
                                                 char **error_json) {
  return guarded(error_json, [&] {
    if (!directory || !config_out)
      invalid("directory and config output are required");
    Loaded ck;
    open_checkpoint(directory, precision ? precision : "bf16", strict != 0, false, ck);
    *config_out = ck.config;
  });
}

extern "C" yuear_status yuear_engine_load(const char *directory, const char *precision,
                                          int32_t strict, yuear_engine **out,
                                          char **error_json) {
  if (out)
    *out = nullptr;
  yuear_status st = guarded(error_json, [&] {
    if (!directory || !out)
      invalid("directory and output pointer are required");
  });
  if (st != YUEAR_SUCCESS)
    return st;
  auto ck = std::make_unique<Loaded>();
  st = guarded(error_json, [&] {
    open_checkpoint(directory, precision ? precision : "bf16", strict != 0, true, *ck);
  });
  if (st != YUEAR_SUCCESS)
    return st;
  yuear_weight_source src{};
  src.kind = YUEAR_WEIGHTS_HOST;
  src.tensors = ck->tensors.data();
  src.count = int32_t(ck->tensors.size());
  const std::string prec = precision ? precision : "bf16";
  src.bits = prec == "8bit" ? 8 : prec == "4bit" ? 4 : 0;
  return yuear_engine_create(&ck->config, &src, out, error_json);
}
