// On-disk checkpoints for the attention path: MLX safetensors files (dense
// f32/f16/bf16 weights, or 8-bit affine layers stored as u32-packed codes
// with f16 scales and biases) and the quantization settings MLX writes into
// config.json. Mirrors CheckpointLoader (checkpoint.rs:480-760): directory
// discovery, quantization detection from the JSON (or YAML) config
// (checkpoint.rs:535-572), falling back to config.json (checkpoint.rs:
// 613-621); and the tensor map `Array::load_safetensors` yields
// (weights.rs:207-237), here mapped from the file without copies.
//
// The safetensors format: an 8-byte little-endian header length N, N bytes
// of JSON {"name": {"dtype", "shape", "data_offsets": [begin, end)}, ...,
// "__metadata__": {...}}, then the data buffer the offsets index.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/relpos_mhsa.h"
#include "host_error.hpp"

namespace {

// ---- a minimal JSON reader (objects, arrays, strings, integers, literals) ----
struct Json {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  bool b = false;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* end;
  bool ok = true;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end - p) < n || std::strncmp(p, s, n)) return false;
    p += n;
    return true;
  }
  std::string string() {
    std::string out;
    if (p >= end || *p != '"') {
      ok = false;
      return out;
    }
    ++p;
    while (p < end && *p != '"') {
      if (*p == '\\' && p + 1 < end) {
        ++p;
        switch (*p) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {  // kept as ASCII when it is, '?' otherwise (names are ASCII)
            unsigned v = 0;
            for (int i = 0; i < 4 && p + 1 < end; ++i) {
              const char c = *++p;
              v = v * 16 + (unsigned)(c >= '0' && c <= '9' ? c - '0' : (c | 32) - 'a' + 10);
            }
            out += v < 128 ? (char)v : '?';
            break;
          }
          default: out += *p;
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= end) ok = false;
    else ++p;
    return out;
  }
  Json value(int depth = 0) {
    Json v;
    ws();
    if (p >= end || depth > 64) {
      ok = false;
      return v;
    }
    if (*p == '{') {
      v.kind = Json::kObj;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return v;
      }
      while (ok) {
        ws();
        std::string k = string();
        ws();
        if (p >= end || *p != ':') {
          ok = false;
          break;
        }
        ++p;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '[') {
      v.kind = Json::kArr;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return v;
      }
      while (ok) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '"') {
      v.kind = Json::kStr;
      v.str = string();
    } else if (lit("true")) {
      v.kind = Json::kBool;
      v.b = true;
    } else if (lit("false")) {
      v.kind = Json::kBool;
    } else if (lit("null")) {
      v.kind = Json::kNull;
    } else {
      char* e = nullptr;
      v.kind = Json::kNum;
      v.num = std::strtod(p, &e);
      if (e == p || e > end) ok = false;
      else p = e;
    }
    return v;
  }
};

bool parse_json(const char* data, size_t n, Json& out) {
  JsonParser ps{data, data + n};
  out = ps.value();
  ps.ws();
  return ps.ok && ps.p == ps.end;
}

int32_t ckfail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return mhsa::set_error(code, buf);
}

bool exists(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0;
}
bool is_dir(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}
bool read_text(const std::string& path, std::string& out) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[65536];
  size_t n;
  out.clear();
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
  std::fclose(f);
  return true;
}

// "quantization": {"bits": N, "group_size": M} from a JSON config, or the
// same mapping in a YAML config (block or flow style); defaults 8 and 64
// (checkpoint.rs:535-572). Returns false when the key is absent.
bool parse_int_after(const std::string& s, const char* key, int& out) {
  const size_t k = s.find(key);
  if (k == std::string::npos) return false;
  size_t i = k + std::strlen(key);
  while (i < s.size() && (s[i] == ' ' || s[i] == '"' || s[i] == '\'' || s[i] == ':')) ++i;
  char* e = nullptr;
  const long v = std::strtol(s.c_str() + i, &e, 10);
  if (e == s.c_str() + i) return false;
  out = (int)v;
  return true;
}

bool parse_quantization(const std::string& text, int& bits, int& group) {
  bits = 8;
  group = 64;
  Json j;
  if (parse_json(text.data(), text.size(), j)) {
    if (j.kind != Json::kObj) return false;
    const Json* q = j.get("quantization");
    if (!q) return false;
    if (const Json* b = q->get("bits"))
      if (b->kind == Json::kNum) bits = (int)b->num;
    if (const Json* g = q->get("group_size"))
      if (g->kind == Json::kNum) group = (int)g->num;
    return true;
  }
  // YAML: a top-level `quantization:` key, its fields on the same line
  // (flow style) or on the indented lines below it
  size_t pos = 0;
  while (pos < text.size()) {
    const size_t eol = std::min(text.find('\n', pos), text.size());
    const std::string line = text.substr(pos, eol - pos);
    if (line.rfind("quantization:", 0) == 0) {
      std::string block = line.substr(13);
      size_t q = eol + 1;
      while (q < text.size()) {
        const size_t e2 = std::min(text.find('\n', q), text.size());
        const std::string l2 = text.substr(q, e2 - q);
        if (!l2.empty() && l2[0] != ' ' && l2[0] != '\t') break;
        block += "\n" + l2;
        q = e2 + 1;
      }
      parse_int_after(block, "bits", bits);
      parse_int_after(block, "group_size", group);
      return true;
    }
    pos = eol + 1;
  }
  return false;
}

int32_t dtype_code(const std::string& s, size_t& esz) {
  if (s == "F32") return esz = 4, MHSA_F32;
  if (s == "F16") return esz = 2, MHSA_F16;
  if (s == "BF16") return esz = 2, MHSA_BF16;
  if (s == "U32") return esz = 4, MHSA_U32;
  return esz = 0, -1;
}

}  // namespace

struct mhsa_checkpoint {
  std::string weights_path;
  int fd = -1;
  void* map = nullptr;
  size_t map_len = 0;
  int quant_bits = 0, quant_group = 0;  // 0 = not quantized
  std::vector<std::string> names;
  std::vector<mhsa_tensor> tensors;                  // name pointers into `names`
  std::vector<std::unique_ptr<char[]>> realigned;    // copies of misaligned tensors
  std::map<std::string, std::string> metadata;
  ~mhsa_checkpoint() {
    if (map && map != MAP_FAILED) ::munmap(map, map_len);
    if (fd >= 0) ::close(fd);
  }
};

extern "C" {

int32_t mhsa_checkpoint_open(const char* path, mhsa_checkpoint** out) {
  if (!path || !out) return ckfail(MHSA_EINVAL, "null argument");
  *out = nullptr;
  std::string weights, config;
  const std::string p(path);
  if (is_dir(p)) {  // checkpoint.rs:694-753
    for (const char* n : {"model.safetensors", "weights.safetensors", "model_weights.safetensors",
                          "weights/model.safetensors"})
      if (weights.empty() && exists(p + "/" + n)) weights = p + "/" + n;
    for (const char* n : {"config.yaml", "model_config.yaml", "config.json", "model_config.json"})
      if (config.empty() && exists(p + "/" + n)) config = p + "/" + n;
    if (weights.empty()) return ckfail(MHSA_ENOENT, "no safetensors weights in %s", path);
  } else {
    weights = p;
    const size_t slash = p.rfind('/');
    const std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
    if (exists(dir + "/config.json")) config = dir + "/config.json";
  }
  std::unique_ptr<mhsa_checkpoint> ck(new (std::nothrow) mhsa_checkpoint());
  if (!ck) return ckfail(MHSA_ENOMEM, "out of host memory");
  ck->weights_path = weights;
  // quantization: the main config, else config.json beside it (checkpoint.rs:613-621)
  std::string text;
  int bits, group;
  bool found = false;
  if (!config.empty() && read_text(config, text)) found = parse_quantization(text, bits, group);
  if (!found && is_dir(p) && exists(p + "/config.json") && read_text(p + "/config.json", text))
    found = parse_quantization(text, bits, group);
  if (found) {
    ck->quant_bits = bits;
    ck->quant_group = group;
  }

  ck->fd = ::open(weights.c_str(), O_RDONLY);
  if (ck->fd < 0) return ckfail(MHSA_ENOENT, "cannot open %s", weights.c_str());
  struct stat st;
  if (::fstat(ck->fd, &st) != 0 || st.st_size < 8) return ckfail(MHSA_EINVAL, "%s is not a safetensors file", weights.c_str());
  ck->map_len = (size_t)st.st_size;
  ck->map = ::mmap(nullptr, ck->map_len, PROT_READ, MAP_PRIVATE, ck->fd, 0);
  if (ck->map == MAP_FAILED) return ckfail(MHSA_ENOMEM, "cannot map %s", weights.c_str());
  const unsigned char* base = static_cast<const unsigned char*>(ck->map);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base[i];
  if (hlen > ck->map_len - 8) return ckfail(MHSA_EINVAL, "%s: header length %llu past the end of the file",
                                            weights.c_str(), (unsigned long long)hlen);
  Json hdr;
  const std::string htext(reinterpret_cast<const char*>(base + 8), (size_t)hlen);  // (NUL-terminated for strtod)
  if (!parse_json(htext.c_str(), htext.size(), hdr) || hdr.kind != Json::kObj)
    return ckfail(MHSA_EINVAL, "%s: malformed safetensors header", weights.c_str());
  const unsigned char* data = base + 8 + hlen;
  const size_t data_len = ck->map_len - 8 - (size_t)hlen;
  ck->names.reserve(hdr.obj.size());
  for (const auto& kv : hdr.obj) {
    if (kv.first == "__metadata__") {
      for (const auto& m : kv.second.obj)
        if (m.second.kind == Json::kStr) ck->metadata[m.first] = m.second.str;
      continue;
    }
    const Json& t = kv.second;
    const Json* dt = t.get("dtype");
    const Json* sh = t.get("shape");
    const Json* off = t.get("data_offsets");
    if (!dt || !sh || !off || dt->kind != Json::kStr || sh->kind != Json::kArr || off->kind != Json::kArr ||
        off->arr.size() != 2)
      return ckfail(MHSA_EINVAL, "%s: bad entry `%s`", weights.c_str(), kv.first.c_str());
    size_t esz;
    const int32_t code = dtype_code(dt->str, esz);
    if (code < 0) continue;  // dtypes the attention path never reads (e.g. int64 counters)
    if (sh->arr.size() > 4) return ckfail(MHSA_ENOTSUP, "`%s`: more than 4 dimensions", kv.first.c_str());
    mhsa_tensor mt{};
    mt.dtype = code;
    mt.ndim = (int32_t)sh->arr.size();
    // dimensions and offsets are whole numbers below 2^53 (exact in the
    // JSON reader's doubles), and the byte size may not wrap: a shape whose
    // product overflows could otherwise match a short data range
    auto whole = [](const Json& j) {
      return j.kind == Json::kNum && j.num >= 0 && j.num < 9.0e15 && j.num == (double)(int64_t)j.num;
    };
    uint64_t nbytes = esz;
    bool ok = whole(off->arr[0]) && whole(off->arr[1]);
    for (size_t i = 0; i < sh->arr.size() && ok; ++i) {
      ok = whole(sh->arr[i]);
      mt.shape[i] = ok ? (int64_t)sh->arr[i].num : 0;
      if (ok && mt.shape[i] && nbytes > data_len / (uint64_t)mt.shape[i] + 1) ok = false;
      nbytes *= (uint64_t)mt.shape[i];
    }
    if (!ok) return ckfail(MHSA_EINVAL, "%s: `%s` has a bad shape or data offsets", weights.c_str(), kv.first.c_str());
    const uint64_t b0 = (uint64_t)off->arr[0].num, b1 = (uint64_t)off->arr[1].num;
    if (b1 < b0 || b1 > data_len || b1 - b0 != nbytes)
      return ckfail(MHSA_EINVAL, "%s: `%s` data offsets do not match its shape", weights.c_str(), kv.first.c_str());
    const unsigned char* src = data + b0;
    if (reinterpret_cast<uintptr_t>(src) % esz) {  // element reads must be aligned
      std::unique_ptr<char[]> copy(new (std::nothrow) char[b1 - b0 + 1]);
      if (!copy) return ckfail(MHSA_ENOMEM, "out of host memory");
      std::memcpy(copy.get(), src, b1 - b0);
      src = reinterpret_cast<const unsigned char*>(copy.get());
      ck->realigned.push_back(std::move(copy));
    }
    mt.data = src;
    ck->names.push_back(kv.first);
    ck->tensors.push_back(mt);
  }
  for (size_t i = 0; i < ck->tensors.size(); ++i) ck->tensors[i].name = ck->names[i].c_str();
  *out = ck.release();
  return MHSA_OK;
}

void mhsa_checkpoint_close(mhsa_checkpoint* ck) { delete ck; }

int32_t mhsa_checkpoint_quantization(const mhsa_checkpoint* ck, int32_t* bits, int32_t* group_size) {
  if (!ck || !bits || !group_size) return ckfail(MHSA_EINVAL, "null argument");
  *bits = ck->quant_bits;
  *group_size = ck->quant_group;
  return MHSA_OK;
}

int32_t mhsa_checkpoint_count(const mhsa_checkpoint* ck) { return ck ? (int32_t)ck->tensors.size() : -1; }

int32_t mhsa_checkpoint_tensor(const mhsa_checkpoint* ck, int32_t idx, mhsa_tensor* out) {
  if (!ck || !out) return ckfail(MHSA_EINVAL, "null argument");
  if (idx < 0 || idx >= (int32_t)ck->tensors.size()) return ckfail(MHSA_EINVAL, "tensor %d out of range", idx);
  *out = ck->tensors[idx];
  return MHSA_OK;
}

int32_t mhsa_checkpoint_metadata(const mhsa_checkpoint* ck, const char* key, const char** value) {
  if (!ck || !key || !value) return ckfail(MHSA_EINVAL, "null argument");
  const auto it = ck->metadata.find(key);
  *value = it == ck->metadata.end() ? nullptr : it->second.c_str();
  return MHSA_OK;
}

int32_t mhsa_load_weights_from_checkpoint(mhsa_layer* layer, const mhsa_checkpoint* ck, const char* prefix,
                                          int32_t strict) {
  if (!ck) return ckfail(MHSA_EINVAL, "null checkpoint");
  // the quantization the checkpoint declares, or (8, 64) (quantization.rs:307)
  return mhsa_load_weights(layer, ck->tensors.data(), (int32_t)ck->tensors.size(), prefix, strict, ck->quant_bits,
                           ck->quant_group);
}

}  // extern "C"
