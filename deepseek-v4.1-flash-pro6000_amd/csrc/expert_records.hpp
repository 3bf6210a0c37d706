// On-disk expert format: the records manifest (components/moe/src/manifest.cpp:35-55
// load_records; written by scripts/assets/expert_bank.py export_tsv), the
// safetensors checkpoint it points into (engine/src/store.cpp:140-217 Store),
// and the check that every record reads exactly the checkpoint's expert
// tensors (engine/src/forward.cu:1781-1832 validate_records, with
// engine/src/store.cpp:79-91 validate_spans). Host code only.
//
// A record is one expert: `bytes` of host buffer filled by its extents (file
// ranges read to dst offsets; a final extent may end at a short EOF as long as
// its `required` bytes arrive), and six views (offset, bytes) into that buffer:
// gate, gate scales, up, up scales, down, down scales (checkpoint names w1, w3,
// w2 .weight / .scale). The kernels read canonical slabs, so a loaded record is
// repacked once into the slab layout of ds41_expert_slab_layout.
#pragma once
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace ds41g {

struct RecordError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

struct RecordView {
  uint64_t offset = 0, bytes = 0;
};
struct RecordExtent {
  std::string path;
  uint64_t file_offset = 0, bytes = 0, dst_offset = 0, required = 0, expected_file_bytes = 0;
  uint64_t need() const { return required ? required : bytes; }
};
struct ExpertRecord {
  uint32_t id = 0;
  uint64_t bytes = 0;
  RecordView view[6];  // gate, gate_scale, up, up_scale, down, down_scale
  std::vector<RecordExtent> extents;
};

// Expert ids of the reference (components/moe/include/ds41/store.hpp:16): 40
// target layers of 384, then 3 drafter layers of 128.
constexpr uint32_t kTargetLayers = 40, kTargetExperts = 384, kDrafterExperts = 128;
constexpr uint32_t kExpertIds = kTargetLayers * kTargetExperts + 3 * kDrafterExperts;

// records manifest: "R id bytes (offset bytes) x 6" and
// "E id \"path\" file_offset bytes dst_offset required expected_file_bytes";
// '#' comments and blank lines are skipped.
inline std::vector<ExpertRecord> parse_records(std::istream &in) {
  std::vector<ExpertRecord> out;
  std::unordered_map<uint32_t, size_t> index;
  std::string line;
  while (std::getline(in, line)) {
    if (line.empty() || line[0] == '#') continue;
    std::istringstream w(line);
    char tag = 0;
    uint32_t id = 0;
    w >> tag >> id;
    if (tag == 'R') {
      ExpertRecord r;
      r.id = id;
      w >> r.bytes;
      for (auto &v : r.view) w >> v.offset >> v.bytes;
      if (!w || id >= kExpertIds || !index.emplace(id, out.size()).second) throw RecordError("bad record line");
      out.push_back(std::move(r));
    } else if (tag == 'E') {
      RecordExtent e;
      w >> std::quoted(e.path) >> e.file_offset >> e.bytes >> e.dst_offset >> e.required >> e.expected_file_bytes;
      auto it = index.find(id);
      if (!w || it == index.end()) throw RecordError("bad extent line");
      out[it->second].extents.push_back(std::move(e));
    } else {
      throw RecordError("unknown manifest line");
    }
  }
  return out;
}

// ---- a small JSON reader for safetensors headers and the shard index ----------
struct JsonValue {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String, or the literal of a Number
  std::vector<JsonValue> items;
  std::vector<std::pair<std::string, JsonValue>> members;
  const JsonValue &at(const std::string &k) const {
    for (const auto &m : members)
      if (m.first == k) return m.second;
    throw RecordError("missing JSON key: " + k);
  }
  uint64_t u64() const {
    if (kind != Number || text.empty() || text[0] == '-' || text.find_first_of(".eE") != std::string::npos)
      throw RecordError("expected an unsigned integer");
    errno = 0;
    char *end = nullptr;
    const unsigned long long v = strtoull(text.c_str(), &end, 10);
    if (errno || *end) throw RecordError("integer out of range");
    return v;
  }
};

class JsonReader {
 public:
  explicit JsonReader(const std::string &s) : s_(s) {}
  JsonValue document() {
    JsonValue v = value(0);
    ws();
    if (i_ != s_.size()) throw RecordError("trailing JSON text");
    return v;
  }

 private:
  const std::string &s_;
  size_t i_ = 0;
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) throw RecordError("truncated JSON");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) throw RecordError(std::string("JSON: expected ") + c);
    ++i_;
  }
  static void utf8(std::string &o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 63));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 63));
      o += (char)(0x80 | (cp & 63));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 63));
      o += (char)(0x80 | ((cp >> 6) & 63));
      o += (char)(0x80 | (cp & 63));
    }
  }
  uint32_t hex4() {
    if (i_ + 4 > s_.size()) throw RecordError("JSON: bad \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else throw RecordError("JSON: bad \\u escape");
    }
    return v;
  }
  std::string str() {
    expect('"');
    std::string o;
    for (;;) {
      if (i_ >= s_.size()) throw RecordError("JSON: unterminated string");
      const char c = s_[i_++];
      if (c == '"') return o;
      if ((unsigned char)c < 0x20) throw RecordError("JSON: control character in string");
      if (c != '\\') {
        o += c;
        continue;
      }
      if (i_ >= s_.size()) throw RecordError("JSON: bad escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && i_ + 1 < s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
            i_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) throw RecordError("JSON: bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, cp);
          break;
        }
        default: throw RecordError("JSON: bad escape");
      }
    }
  }
  JsonValue value(int depth) {
    if (depth > 64) throw RecordError("JSON nested too deeply");
    JsonValue v;
    const char c = peek();
    if (c == '{') {
      ++i_;
      v.kind = JsonValue::Object;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      for (;;) {
        std::string k = str();
        expect(':');
        v.members.emplace_back(std::move(k), value(depth + 1));
        if (peek() == ',') {
          ++i_;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      ++i_;
      v.kind = JsonValue::Array;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      for (;;) {
        v.items.push_back(value(depth + 1));
        if (peek() == ',') {
          ++i_;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = JsonValue::String;
      v.text = str();
      return v;
    }
    if (s_.compare(i_, 4, "true") == 0 || s_.compare(i_, 5, "false") == 0) {
      v.kind = JsonValue::Bool;
      v.b = s_[i_] == 't';
      i_ += v.b ? 4 : 5;
      return v;
    }
    if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
      return v;
    }
    const size_t start = i_;
    while (i_ < s_.size() && (isdigit((unsigned char)s_[i_]) || strchr("+-.eE", s_[i_]))) ++i_;
    if (start == i_) throw RecordError("JSON: unexpected character");
    v.kind = JsonValue::Number;
    v.text = s_.substr(start, i_ - start);
    return v;
  }
};

// ---- the safetensors checkpoint ------------------------------------------------
struct CkptTensor {
  std::string name, path, dtype;
  std::vector<uint64_t> shape;
  uint64_t offset = 0, bytes = 0, file_bytes = 0;
};

inline uint64_t add_checked(uint64_t a, uint64_t b) {
  if (a > UINT64_MAX - b) throw RecordError("tensor offset overflow");
  return a + b;
}
inline uint64_t mul_checked(uint64_t a, uint64_t b) {
  if (b && a > UINT64_MAX / b) throw RecordError("tensor shape overflow");
  return a * b;
}

inline void pread_exact(int fd, void *dst, uint64_t n, uint64_t off) {
  uint64_t done = 0;
  while (done < n) {
    const ssize_t r = pread(fd, static_cast<char *>(dst) + done, n - done, (off_t)(off + done));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) throw RecordError("short read");
    done += (uint64_t)r;
  }
}

struct Fd {
  int fd;
  explicit Fd(const std::string &p) : fd(open(p.c_str(), O_RDONLY | O_CLOEXEC)) {
    if (fd < 0) throw RecordError("open failed: " + p);
  }
  ~Fd() { close(fd); }
  Fd(const Fd &) = delete;
  Fd &operator=(const Fd &) = delete;
};

// Checkpoint tensor names as the engine binds them (engine/src/store.cpp:124-139).
inline std::string normalize_tensor_name(std::string n) {
  if (n.rfind("model.", 0) == 0) n.erase(0, 6);
  auto swap_all = [&](const std::string &a, const std::string &b) {
    for (size_t i = 0; (i = n.find(a, i)) != std::string::npos; i += b.size()) n.replace(i, a.size(), b);
  };
  swap_all("self_attn", "attn");
  if (n.rfind("vision.", 0) != 0) swap_all("mlp", "ffn");
  swap_all("weight_scale_inv", "scale");
  swap_all("e_score_correction_bias", "bias");
  return n;
}

inline uint64_t dtype_bytes(const std::string &d) {
  static const std::map<std::string, uint64_t> size = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"I16", 2},     {"I32", 4},       {"I64", 8},     {"F16", 2},
      {"BF16", 2}, {"F32", 4}, {"F64", 8}, {"F8_E4M3", 1}, {"F8_E4M3FN", 1}, {"F8_E8M0", 1}, {"F8_E8M0FNU", 1}};
  auto it = size.find(d);
  if (it == size.end()) throw RecordError("unsupported native dtype " + d);
  return it->second;
}

// Opens model.safetensors.index.json under root and every shard it names: each
// header is checked (length, dtype, shape x dtype == range, data ranges tile
// [0, end) without gaps or overlap) and, with `complete`, each file must be
// exactly 8 + header + data bytes long.
inline std::map<std::string, CkptTensor> open_checkpoint(const std::string &root_in, bool complete) {
  namespace fs = std::filesystem;
  const fs::path root = fs::canonical(root_in);
  std::ifstream f(root / "model.safetensors.index.json");
  if (!f) throw RecordError("cannot open " + (root / "model.safetensors.index.json").string());
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string index_text = ss.str();
  const JsonValue index = JsonReader(index_text).document();
  const JsonValue &map = index.at("weight_map");
  if (map.kind != JsonValue::Object) throw RecordError("weight_map is not an object");
  struct Shard {
    JsonValue header;
    uint64_t start = 0, file_bytes = 0;
    std::string path;
  };
  std::map<std::string, Shard> shards;
  std::map<std::string, CkptTensor> out;
  for (const auto &m : map.members) {
    if (m.second.kind != JsonValue::String) throw RecordError("weight_map value is not a string");
    const std::string &shard = m.second.text;
    const fs::path rel(shard);
    if (rel.is_absolute() || rel.filename() != rel) throw RecordError("unsafe shard path");
    if (!shards.count(shard)) {
      Shard sh;
      sh.path = (root / rel).string();
      Fd fd(sh.path);
      uint8_t lb[8];
      pread_exact(fd.fd, lb, 8, 0);
      uint64_t len = 0;
      for (int k = 0; k < 8; ++k) len |= (uint64_t)lb[k] << (8 * k);
      if (!len || len > (128ull << 20)) throw RecordError("invalid safetensors header length");
      std::string raw(len, '\0');
      pread_exact(fd.fd, raw.data(), len, 8);
      sh.header = JsonReader(raw).document();
      if (sh.header.kind != JsonValue::Object) throw RecordError("safetensors header is not an object");
      sh.start = add_checked(8, len);
      uint64_t end = 0;
      std::vector<std::pair<uint64_t, uint64_t>> ranges;
      for (const auto &t : sh.header.members) {
        if (t.first == "__metadata__") continue;
        const JsonValue &r = t.second.at("data_offsets");
        if (r.items.size() != 2 || r.items[1].u64() < r.items[0].u64()) throw RecordError("invalid tensor range");
        uint64_t bytes = dtype_bytes(t.second.at("dtype").text);
        for (const auto &d : t.second.at("shape").items) bytes = mul_checked(bytes, d.u64());
        const uint64_t lo = r.items[0].u64(), hi = r.items[1].u64();
        if (bytes != hi - lo) throw RecordError("tensor byte/shape mismatch: " + t.first);
        if (bytes) ranges.push_back({lo, hi});
        end = std::max(end, hi);
      }
      std::sort(ranges.begin(), ranges.end());
      uint64_t cursor = 0;
      for (const auto &r : ranges) {
        if (r.first != cursor) throw RecordError("overlapping or gapped tensor data");
        cursor = r.second;
      }
      struct stat st{};
      if (fstat(fd.fd, &st)) throw RecordError("fstat failed");
      sh.file_bytes = add_checked(sh.start, end);
      if (complete && (uint64_t)st.st_size != sh.file_bytes) throw RecordError("incomplete/changed shard: " + shard);
      shards.emplace(shard, std::move(sh));
    }
    const Shard &sh = shards.at(shard);
    const JsonValue &d = sh.header.at(m.first);
    const JsonValue &r = d.at("data_offsets");
    CkptTensor t;
    t.name = normalize_tensor_name(m.first);
    t.path = sh.path;
    t.dtype = d.at("dtype").text;
    for (const auto &x : d.at("shape").items) t.shape.push_back(x.u64());
    t.offset = add_checked(sh.start, r.items.at(0).u64());
    t.bytes = r.items.at(1).u64() - r.items.at(0).u64();
    t.file_bytes = sh.file_bytes;
    const std::string name = t.name;
    if (!out.emplace(name, std::move(t)).second) throw RecordError("duplicate normalized name: " + name);
  }
  return out;
}

// Record extents: non-empty, inside the record, sorted without overlap.
inline void check_spans(uint64_t size, std::vector<std::pair<uint64_t, uint64_t>> spans) {
  if (!size || spans.empty()) throw RecordError("empty expert record/spans");
  std::sort(spans.begin(), spans.end());
  uint64_t end = 0;
  for (const auto &s : spans) {
    if (!s.second || s.first < end || s.first > size || s.second > size - s.first)
      throw RecordError("overlapping/out-of-bounds expert read spans");
    end = s.first + s.second;
  }
}

inline std::string expert_prefix(uint32_t id) {
  const uint32_t base = kTargetLayers * kTargetExperts;
  const uint32_t layer = id < base ? id / kTargetExperts : kTargetLayers + (id - base) / kDrafterExperts;
  const uint32_t e = id < base ? id % kTargetExperts : (id - base) % kDrafterExperts;
  return (layer < kTargetLayers ? "layers." + std::to_string(layer) : "mtp." + std::to_string(layer - kTargetLayers)) +
         ".ffn.experts." + std::to_string(e);
}

// Every record must read exactly the checkpoint's six expert tensors: each
// view has the tensor's byte count and lies inside the required part of an
// extent of the tensor's own file at the tensor's own file offset, and every
// extent serves at least one view.
inline void validate_records(const std::vector<ExpertRecord> &records,
                             const std::map<std::string, CkptTensor> &ckpt) {
  static const char *kField[6] = {"w1.weight", "w1.scale", "w3.weight", "w3.scale", "w2.weight", "w2.scale"};
  std::vector<char> seen(kExpertIds, 0);
  for (const auto &r : records) {
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    for (const auto &e : r.extents) {
      if (e.need() > e.bytes || e.file_offset > e.expected_file_bytes ||
          e.need() > e.expected_file_bytes - e.file_offset)
        throw RecordError("invalid required expert span/file coverage");
      spans.emplace_back(e.dst_offset, e.bytes);
    }
    check_spans(r.bytes, spans);
    if (r.id >= kExpertIds || seen[r.id]) throw RecordError("expert manifest duplicate/id");
    seen[r.id] = 1;
    const std::string prefix = expert_prefix(r.id);
    std::vector<char> used(r.extents.size(), 0);
    for (int f = 0; f < 6; ++f) {
      auto it = ckpt.find(prefix + "." + kField[f]);
      if (it == ckpt.end()) throw RecordError("missing checkpoint tensor " + prefix + "." + kField[f]);
      const CkptTensor &t = it->second;
      const RecordView &v = r.view[f];
      if (v.bytes != t.bytes) throw RecordError("expert view byte mismatch");
      bool found = false;
      for (size_t k = 0; k < r.extents.size(); ++k) {
        const RecordExtent &e = r.extents[k];
        const uint64_t cover = e.need();
        if (v.offset >= e.dst_offset && v.offset - e.dst_offset <= cover && v.bytes <= cover - (v.offset - e.dst_offset) &&
            e.path == t.path && e.expected_file_bytes == t.file_bytes &&
            e.file_offset + (v.offset - e.dst_offset) == t.offset)
          found = used[k] = 1;
      }
      if (!found) throw RecordError("expert view does not match verified native tensor/required extent coverage: " + prefix);
    }
    if (std::find(used.begin(), used.end(), 0) != used.end()) throw RecordError("extraneous expert read span");
  }
}

// Reads a record's extents into dst (record.bytes bytes). An extent may end at
// EOF before `bytes` (its file is shorter than the aligned read) as long as its
// required bytes arrived; the rest of the extent is zeroed.
inline void read_record(const ExpertRecord &r, uint8_t *dst) {
  for (const auto &e : r.extents) {
    Fd fd(e.path);
    struct stat st{};
    if (fstat(fd.fd, &st)) throw RecordError("fstat failed");
    if ((uint64_t)st.st_size != e.expected_file_bytes) throw RecordError("expert file size changed: " + e.path);
    uint64_t done = 0;
    while (done < e.bytes) {
      const ssize_t n = pread(fd.fd, dst + e.dst_offset + done, e.bytes - done, (off_t)(e.file_offset + done));
      if (n < 0 && errno == EINTR) continue;
      if (n < 0) throw RecordError("read failed: " + e.path);
      if (n == 0) break;
      done += (uint64_t)n;
    }
    if (done < e.need()) throw RecordError("short expert read: " + e.path);
    if (done < e.bytes) memset(dst + e.dst_offset + done, 0, e.bytes - done);
  }
}

}  // namespace ds41g
