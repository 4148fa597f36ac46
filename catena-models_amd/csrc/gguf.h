// GGUF checkpoints (src/checkpoint.rs): version-3 files, a single file, any
// member of a standard shard set (<prefix>-NNNNN-of-MMMMM.gguf) or a
// directory of .gguf files; model configuration from the metadata
// (parse_gguf_model_config, checkpoint.rs:422-639); tensor inventory, shapes,
// dtypes and byte ranges checked against weight_specs (validate_files,
// checkpoint.rs:659-733; tensor_view, 766-820). Host code only: the payloads
// are mapped read-only and handed to cq35_model_create, which copies them
// into HBM (the reference maps them into the GPU address space instead).
#pragma once

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

namespace cq35 {
namespace gguf {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
enum : uint32_t { kF32 = 0, kF16 = 1, kBF16 = 30 };
enum ValueType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7,
  STRING = 8, ARRAY = 9, U64 = 10, I64 = 11, F64 = 12
};

struct Tensor {
  std::vector<uint64_t> dims;  // outermost first (the file stores innermost first)
  uint32_t type = 0;
  uint64_t offset = 0;         // absolute file offset of the payload
  int file = 0;
};

struct Scalar {
  bool is_float = false;
  double f = 0.0;
  uint64_t u = 0;
};

struct File {
  std::string path;
  const uint8_t* base = nullptr;
  size_t size = 0;
  ~File() {
    if (base) munmap(const_cast<uint8_t*>(base), size);
  }
};

struct Checkpoint {
  std::vector<File*> files;
  std::map<std::string, Tensor> tensors;
  std::string arch;
  std::map<std::string, Scalar> scalars;  // architecture-scoped numeric keys
  uint64_t token_count = 0;               // tokenizer.ggml.tokens length
  bool has_tokens = false;
  ~Checkpoint() {
    for (File* f : files) delete f;
  }
};

class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return pos_; }
  bool take(size_t k, const uint8_t** out) {
    if (n_ - pos_ < k) return false;
    if (out) *out = p_ + pos_;
    pos_ += k;
    return true;
  }
  bool u32(uint32_t* v) {
    const uint8_t* q;
    if (!take(4, &q)) return false;
    std::memcpy(v, q, 4);
    return true;
  }
  bool u64(uint64_t* v) {
    const uint8_t* q;
    if (!take(8, &q)) return false;
    std::memcpy(v, q, 8);
    return true;
  }
  bool str(std::string* s) {
    uint64_t len;
    const uint8_t* q;
    if (!u64(&len) || len > (1ull << 30) || !take((size_t)len, &q)) return false;
    s->assign(reinterpret_cast<const char*>(q), (size_t)len);
    return true;
  }
  bool skip(uint32_t type, int depth) {
    if (depth > 8) return false;
    switch (type) {
      case U8: case I8: case BOOL: return take(1, nullptr);
      case U16: case I16: return take(2, nullptr);
      case U32: case I32: case F32: return take(4, nullptr);
      case U64: case I64: case F64: return take(8, nullptr);
      case STRING: {
        uint64_t len;
        return u64(&len) && len <= (1ull << 30) && take((size_t)len, nullptr);
      }
      case ARRAY: {
        uint32_t et;
        uint64_t len;
        if (!u32(&et) || !u64(&len) || len > 10000000ull) return false;
        for (uint64_t i = 0; i < len; ++i)
          if (!skip(et, depth + 1)) return false;
        return true;
      }
      default: return false;
    }
  }
  // integer or float scalar
  bool scalar(uint32_t type, Scalar* out) {
    const uint8_t* q;
    switch (type) {
      case U8: case BOOL: if (!take(1, &q)) return false; out->u = q[0]; return true;
      case I8: if (!take(1, &q)) return false; if ((int8_t)q[0] < 0) return false; out->u = q[0]; return true;
      case U16: { uint16_t v; if (!take(2, &q)) return false; std::memcpy(&v, q, 2); out->u = v; return true; }
      case I16: { int16_t v; if (!take(2, &q)) return false; std::memcpy(&v, q, 2); if (v < 0) return false; out->u = (uint64_t)v; return true; }
      case U32: { uint32_t v; if (!u32(&v)) return false; out->u = v; return true; }
      case I32: { int32_t v; if (!take(4, &q)) return false; std::memcpy(&v, q, 4); if (v < 0) return false; out->u = (uint64_t)v; return true; }
      case U64: return u64(&out->u);
      case I64: { int64_t v; if (!take(8, &q)) return false; std::memcpy(&v, q, 8); if (v < 0) return false; out->u = (uint64_t)v; return true; }
      case F32: { float v; if (!take(4, &q)) return false; std::memcpy(&v, q, 4); out->is_float = true; out->f = v; return true; }
      case F64: { double v; if (!take(8, &q)) return false; std::memcpy(&v, q, 8); out->is_float = true; out->f = v; return true; }
      default: return false;
    }
  }

 private:
  const uint8_t* p_;
  size_t n_;
  size_t pos_ = 0;
};

// The numeric metadata keys the configuration reads (is_model_scalar_key,
// checkpoint.rs:641-669), without the architecture prefix.
inline bool model_scalar_suffix(const std::string& key, const std::string& arch) {
  static const char* kSuffixes[] = {
      "vocab_size", "embedding_length", "feed_forward_length", "expert_feed_forward_length",
      "block_count", "nextn_predict_layers", "attention.head_count", "attention.head_count_kv",
      "attention.key_length", "context_length", "attention.layer_norm_rms_epsilon",
      "rope.freq_base", "rope.dimension_count", "expert_count", "expert_used_count",
      "expert_shared_feed_forward_length", "full_attention_interval", "ssm.conv_kernel",
      "ssm.state_size", "ssm.group_count", "ssm.time_step_rank", "ssm.inner_size"};
  if (key.compare(0, arch.size() + 1, arch + ".") != 0) return false;
  const std::string rest = key.substr(arch.size() + 1);
  for (const char* s : kSuffixes)
    if (rest == s) return true;
  return false;
}

// The files a path names (resolve_gguf_paths, checkpoint.rs:263-324).
inline bool resolve(const std::string& path, std::vector<std::string>* out, std::string* err) {
  struct stat st;
  if (stat(path.c_str(), &st) != 0) { *err = "cannot stat " + path; return false; }
  out->clear();
  if (S_ISDIR(st.st_mode)) {
    DIR* d = opendir(path.c_str());
    if (!d) { *err = "cannot read directory " + path; return false; }
    while (dirent* e = readdir(d)) {
      std::string name = e->d_name;
      if (name.size() > 5) {
        std::string ext = name.substr(name.size() - 5);
        std::transform(ext.begin(), ext.end(), ext.begin(), ::tolower);
        if (ext == ".gguf") out->push_back(path + "/" + name);
      }
    }
    closedir(d);
    std::sort(out->begin(), out->end());
    if (out->empty()) { *err = "directory " + path + " contains no .gguf files"; return false; }
    return true;
  }
  // <prefix>-NNNNN-of-MMMMM.gguf: every shard of the set
  const size_t slash = path.rfind('/');
  const std::string dir = slash == std::string::npos ? "" : path.substr(0, slash + 1);
  const std::string file = slash == std::string::npos ? path : path.substr(slash + 1);
  const std::string suffix = ".gguf";
  if (file.size() > suffix.size() && file.compare(file.size() - suffix.size(), suffix.size(), suffix) == 0) {
    const std::string stem = file.substr(0, file.size() - suffix.size());
    const size_t of = stem.rfind("-of-");
    if (of != std::string::npos) {
      const size_t dash = stem.rfind('-', of - 1);
      const std::string index = dash == std::string::npos ? "" : stem.substr(dash + 1, of - dash - 1);
      const std::string total = stem.substr(of + 4);
      auto digits = [](const std::string& s) {
        return !s.empty() && std::all_of(s.begin(), s.end(), [](char c) { return c >= '0' && c <= '9'; });
      };
      if (dash != std::string::npos && digits(index) && digits(total)) {
        const long idx = std::stol(index), tot = std::stol(total);
        if (idx < 1 || tot < 1 || idx > tot || tot > 100000) {
          *err = "invalid GGUF shard " + index + " of " + total + " in " + path;
          return false;
        }
        const std::string prefix = stem.substr(0, dash);
        for (long sh = 1; sh <= tot; ++sh) {
          std::string num = std::to_string(sh);
          if (num.size() < index.size()) num = std::string(index.size() - num.size(), '0') + num;
          out->push_back(dir + prefix + "-" + num + "-of-" + total + suffix);
        }
        return true;
      }
    }
  }
  out->push_back(path);
  return true;
}

// Map one file and parse its header: metadata (architecture, numeric keys,
// tokenizer size, alignment) and tensor infos (parse_gguf,
// checkpoint.rs:1181-1261).
inline bool open_file(const std::string& path, int index, Checkpoint* ck, std::string* err) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) { *err = "cannot open " + path; return false; }
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    *err = path + " is too short for a GGUF header";
    return false;
  }
  void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) { *err = "cannot map " + path; return false; }
  File* f = new File();
  f->path = path;
  f->base = static_cast<const uint8_t*>(map);
  f->size = (size_t)st.st_size;
  ck->files.push_back(f);
  Cursor c(f->base, f->size);
  auto bad = [&](const std::string& what) { *err = path + ": " + what; return false; };
  uint32_t magic, version;
  uint64_t tensor_count, meta_count;
  if (!c.u32(&magic) || magic != kMagic) return bad("file does not have GGUF magic");
  if (!c.u32(&version) || version != kVersion) return bad("only GGUF version 3 is supported");
  if (!c.u64(&tensor_count) || !c.u64(&meta_count)) return bad("truncated header");
  if (tensor_count > 1000000 || meta_count > 1000000) return bad("unreasonable tensor or metadata count");
  uint64_t alignment = kDefaultAlignment;
  std::string arch;
  std::vector<std::pair<std::string, Scalar>> numeric;
  for (uint64_t i = 0; i < meta_count; ++i) {
    std::string key;
    uint32_t type;
    if (!c.str(&key) || !c.u32(&type)) return bad("truncated metadata");
    if (key == "general.alignment") {
      Scalar s;
      if (!c.scalar(type, &s) || s.is_float) return bad("general.alignment is not an unsigned integer");
      alignment = s.u;
    } else if (key == "general.architecture") {
      if (type != STRING || !c.str(&arch)) return bad("general.architecture is not a string");
    } else if (key == "tokenizer.ggml.tokens" && index == 0) {
      uint32_t et;
      uint64_t len;
      if (type != ARRAY || !c.u32(&et) || et != STRING || !c.u64(&len))
        return bad("tokenizer.ggml.tokens is not a string array");
      for (uint64_t k = 0; k < len; ++k)
        if (!c.skip(STRING, 1)) return bad("truncated tokenizer tokens");
      ck->token_count = len;
      ck->has_tokens = true;
    } else if (type != ARRAY && type != STRING && type != BOOL) {
      Scalar s;
      if (!c.scalar(type, &s)) return bad("malformed metadata value for " + key);
      numeric.emplace_back(key, s);
    } else if (!c.skip(type, 0)) {
      return bad("malformed metadata value for " + key);
    }
  }
  if (alignment == 0 || (alignment & (alignment - 1)) != 0)
    return bad("alignment is not a positive power of two");
  if (index == 0) {
    ck->arch = arch;
    for (auto& kv : numeric)
      if (!arch.empty() && model_scalar_suffix(kv.first, arch))
        ck->scalars[kv.first.substr(arch.size() + 1)] = kv.second;
  }
  std::vector<std::pair<std::string, Tensor>> infos;
  for (uint64_t i = 0; i < tensor_count; ++i) {
    std::string name;
    uint32_t nd;
    if (!c.str(&name) || !c.u32(&nd) || nd > 8) return bad("malformed tensor info");
    Tensor t;
    t.dims.resize(nd);
    for (uint32_t k = 0; k < nd; ++k)
      if (!c.u64(&t.dims[nd - 1 - k])) return bad("truncated tensor info");
    uint64_t rel;
    if (!c.u32(&t.type) || !c.u64(&rel)) return bad("truncated tensor info");
    if (t.type != kF32 && t.type != kF16 && t.type != kBF16)
      return bad("tensor " + name + " has unsupported type " + std::to_string(t.type) + "; expected F32, BF16 or F16");
    if (rel % alignment) return bad("tensor " + name + " offset is not aligned");
    t.offset = rel;
    t.file = index;
    infos.emplace_back(name, t);
  }
  const uint64_t data_start = ((uint64_t)c.pos() + alignment - 1) & ~(alignment - 1);
  if (data_start > f->size) return bad("tensor data begins beyond the end of the file");
  for (auto& it : infos) {
    it.second.offset += data_start;
    if (!ck->tensors.emplace(it.first, it.second).second)
      return bad("duplicate GGUF tensor " + it.first);
  }
  return true;
}

inline bool open_all(const std::string& path, Checkpoint* ck, std::string* err) {
  std::vector<std::string> paths;
  if (!resolve(path, &paths, err)) return false;
  for (size_t i = 0; i < paths.size(); ++i)
    if (!open_file(paths[i], (int)i, ck, err)) return false;
  return true;
}

}  // namespace gguf
}  // namespace cq35
