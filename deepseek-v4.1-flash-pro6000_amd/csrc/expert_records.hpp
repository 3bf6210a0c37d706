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
#include <iterator>
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

// ---- byte ranges ---------------------------------------------------------------
struct Range {
  uint64_t lo = 0, len = 0;
};
// inner lies within outer (an empty inner may sit at outer's end).
inline bool range_within(const Range &outer, const Range &inner) {
  if (inner.lo < outer.lo) return false;
  const uint64_t rel = inner.lo - outer.lo;
  return rel <= outer.len && inner.len <= outer.len - rel;
}
// Sorted by start (then length), every range begins exactly where the previous
// one ends, the first at 0: together they cover [0, end) once.
inline bool ranges_tile_from_zero(std::vector<Range> v) {
  std::sort(v.begin(), v.end(), [](const Range &x, const Range &y) { return x.lo < y.lo || (x.lo == y.lo && x.len < y.len); });
  if (!v.empty() && v.front().lo != 0) return false;
  return std::adjacent_find(v.begin(), v.end(), [](const Range &x, const Range &y) { return y.lo != x.lo + x.len; }) ==
         v.end();
}
// No two non-empty ranges share a byte.
inline bool ranges_disjoint(std::vector<Range> v) {
  std::sort(v.begin(), v.end(), [](const Range &x, const Range &y) { return x.lo < y.lo || (x.lo == y.lo && x.len < y.len); });
  return std::adjacent_find(v.begin(), v.end(), [](const Range &x, const Range &y) { return y.lo - x.lo < x.len; }) ==
         v.end();
}
inline uint64_t sum_or_throw(uint64_t a, uint64_t b, const char *what) {
  uint64_t r;
  if (__builtin_add_overflow(a, b, &r)) throw RecordError(std::string(what) + ": 64-bit overflow");
  return r;
}
inline uint64_t product_or_throw(uint64_t a, uint64_t b, const char *what) {
  uint64_t r;
  if (__builtin_mul_overflow(a, b, &r)) throw RecordError(std::string(what) + ": 64-bit overflow");
  return r;
}

inline void pread_exact(int fd, void *dst, uint64_t n, uint64_t off) {
  for (uint64_t done = 0; done < n;) {
    const ssize_t r = pread(fd, static_cast<char *>(dst) + done, n - done, (off_t)(off + done));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) throw RecordError(r == 0 ? "file ends before the bytes it must hold" : "read error");
    done += (uint64_t)r;
  }
}

struct Fd {
  int fd;
  explicit Fd(const std::string &p) : fd(open(p.c_str(), O_RDONLY | O_CLOEXEC)) {
    if (fd < 0) throw RecordError("cannot open " + p);
  }
  ~Fd() { close(fd); }
  Fd(const Fd &) = delete;
  Fd &operator=(const Fd &) = delete;
  uint64_t size() const {
    struct stat st{};
    if (fstat(fd, &st)) throw RecordError("cannot stat an open file");
    return (uint64_t)st.st_size;
  }
};

// ---- the safetensors checkpoint ------------------------------------------------
// Where a checkpoint tensor's bytes are: its file, that file's full size, and
// the absolute offset and length of the tensor in it.
struct CkptTensor {
  std::string name, path, dtype;
  std::vector<uint64_t> shape;
  uint64_t offset = 0, bytes = 0, file_bytes = 0;
};

// The tensor names the engine binds (engine/src/store.cpp:124-139): "model."
// dropped, then each rewrite applied left to right over the whole name.
inline std::string checkpoint_name(std::string n) {
  static const std::string model = "model.", vision = "vision.";
  if (n.compare(0, model.size(), model) == 0) n.erase(0, model.size());
  struct Rewrite {
    const char *from, *to;
    bool outside_vision_only;
  };
  static const Rewrite rewrites[] = {{"self_attn", "attn", false},
                                     {"mlp", "ffn", true},
                                     {"weight_scale_inv", "scale", false},
                                     {"e_score_correction_bias", "bias", false}};
  for (const Rewrite &rw : rewrites) {
    if (rw.outside_vision_only && n.compare(0, vision.size(), vision) == 0) continue;
    const std::string from = rw.from, to = rw.to;
    std::string out;
    size_t at = 0;
    for (size_t hit; (hit = n.find(from, at)) != std::string::npos; at = hit + from.size()) out.append(n, at, hit - at).append(to);
    n = out.append(n, at, std::string::npos);
  }
  return n;
}

// Element sizes of the safetensors dtypes the engine accepts.
inline uint64_t element_bytes(const std::string &dtype) {
  static const std::unordered_map<std::string, uint64_t> table = {
      {"BOOL", 1}, {"U8", 1}, {"I8", 1}, {"F8_E4M3", 1}, {"F8_E4M3FN", 1}, {"F8_E8M0", 1}, {"F8_E8M0FNU", 1},
      {"I16", 2},  {"F16", 2}, {"BF16", 2}, {"I32", 4}, {"F32", 4}, {"I64", 8}, {"F64", 8}};
  const auto it = table.find(dtype);
  if (it == table.end()) throw RecordError("dtype " + dtype + " is not one the engine reads");
  return it->second;
}

// One shard: its header, where its data starts, and the size the file has when
// complete (data start + the furthest tensor end).
struct ShardScan {
  JsonValue header;
  uint64_t data_start = 0, file_bytes = 0;
  std::string path;
};

// A shard's header must be 1 byte .. 128 MiB of JSON object; each tensor entry
// (all but __metadata__) has a known dtype, an unsigned shape and a [lo, hi]
// range whose length is the shape's byte count; the non-empty ranges cover
// [0, end) exactly once. With `complete`, the file is data start + end bytes.
inline ShardScan scan_shard(const std::string &path, bool complete) {
  ShardScan sh;
  sh.path = path;
  Fd fd(path);
  uint8_t le[8];
  pread_exact(fd.fd, le, sizeof le, 0);
  uint64_t header_len = 0;
  for (int k = 7; k >= 0; --k) header_len = (header_len << 8) | le[k];
  if (header_len == 0 || header_len > (128ull << 20)) throw RecordError("shard header length out of range: " + path);
  std::string text(header_len, '\0');
  pread_exact(fd.fd, &text[0], header_len, sizeof le);
  sh.header = JsonReader(text).document();
  if (sh.header.kind != JsonValue::Object) throw RecordError("shard header is not a JSON object: " + path);
  std::vector<Range> data;
  uint64_t end = 0;
  for (const auto &entry : sh.header.members) {
    if (entry.first == "__metadata__") continue;
    const JsonValue &lohi = entry.second.at("data_offsets"), &shape = entry.second.at("shape");
    if (lohi.kind != JsonValue::Array || lohi.items.size() != 2 || shape.kind != JsonValue::Array)
      throw RecordError("tensor entry without a [lo, hi] range or a shape: " + entry.first);
    const uint64_t lo = lohi.items[0].u64(), hi = lohi.items[1].u64();
    if (hi < lo) throw RecordError("tensor range ends before it starts: " + entry.first);
    uint64_t need = element_bytes(entry.second.at("dtype").text);
    for (const auto &dim : shape.items) need = product_or_throw(need, dim.u64(), "tensor size");
    if (need != hi - lo) throw RecordError("tensor range does not hold its shape and dtype: " + entry.first);
    if (need) data.push_back(Range{lo, need});
    end = std::max(end, hi);
  }
  if (!ranges_tile_from_zero(data)) throw RecordError("tensor data of the shard has gaps or overlaps: " + path);
  sh.data_start = sum_or_throw(sizeof le, header_len, "shard data start");
  sh.file_bytes = sum_or_throw(sh.data_start, end, "shard size");
  const uint64_t have = fd.size();
  if (complete && have != sh.file_bytes)
    throw RecordError("shard is incomplete or was changed: " + path + " holds " + std::to_string(have) +
                      " bytes, its header describes " + std::to_string(sh.file_bytes));
  return sh;
}

// A shard file name from the index: one path component, relative.
inline bool plain_file_name(const std::string &s) {
  const std::filesystem::path p(s);
  return !s.empty() && !p.is_absolute() && p == p.filename();
}

// Every tensor of the checkpoint under root (model.safetensors.index.json and
// the shards it names, each scanned once), by its engine name; two source
// names that become one engine name are an error.
inline std::map<std::string, CkptTensor> open_checkpoint(const std::string &root_in, bool complete) {
  namespace fs = std::filesystem;
  const fs::path root = fs::canonical(root_in);
  const fs::path index_path = root / "model.safetensors.index.json";
  std::ifstream f(index_path);
  if (!f) throw RecordError("cannot open " + index_path.string());
  const std::string index_text((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  const JsonValue index = JsonReader(index_text).document();
  const JsonValue &weight_map = index.at("weight_map");
  if (weight_map.kind != JsonValue::Object) throw RecordError("weight_map must be a JSON object");
  std::map<std::string, ShardScan> scanned;
  std::map<std::string, CkptTensor> tensors;
  for (const auto &entry : weight_map.members) {
    if (entry.second.kind != JsonValue::String || !plain_file_name(entry.second.text))
      throw RecordError("weight_map names a shard outside the checkpoint directory: " + entry.first);
    const std::string &shard = entry.second.text;
    auto it = scanned.find(shard);
    if (it == scanned.end()) it = scanned.emplace(shard, scan_shard((root / shard).string(), complete)).first;
    const ShardScan &sh = it->second;
    const JsonValue &desc = sh.header.at(entry.first);
    const JsonValue &lohi = desc.at("data_offsets");
    CkptTensor t;
    t.name = checkpoint_name(entry.first);
    t.path = sh.path;
    t.dtype = desc.at("dtype").text;
    for (const auto &dim : desc.at("shape").items) t.shape.push_back(dim.u64());
    t.offset = sum_or_throw(sh.data_start, lohi.items.at(0).u64(), "tensor offset");
    t.bytes = lohi.items.at(1).u64() - lohi.items.at(0).u64();
    t.file_bytes = sh.file_bytes;
    if (tensors.count(t.name)) throw RecordError("two checkpoint tensors share the engine name " + t.name);
    tensors.emplace(t.name, std::move(t));
  }
  return tensors;
}

// ---- records against the checkpoint ------------------------------------------
// A record's buffer geometry: some bytes and extents, each extent non-empty,
// inside the buffer, and no two extents writing the same byte.
inline void check_destinations(const ExpertRecord &r) {
  if (r.bytes == 0 || r.extents.empty()) throw RecordError("expert record without bytes or extents");
  std::vector<Range> dst;
  for (const auto &e : r.extents) {
    const Range d{e.dst_offset, e.bytes};
    if (d.len == 0 || !range_within(Range{0, r.bytes}, d))
      throw RecordError("expert extent is empty or lies outside its record buffer");
    dst.push_back(d);
  }
  if (!ranges_disjoint(dst)) throw RecordError("expert extents overlap in the record buffer");
}

// The checkpoint name of one of a record's six tensors (ids as in
// components/moe/include/ds41/store.hpp:16).
inline std::string expert_tensor_name(uint32_t id, int field) {
  static const char *kField[6] = {"w1.weight", "w1.scale", "w3.weight", "w3.scale", "w2.weight", "w2.scale"};
  constexpr uint32_t target_ids = kTargetLayers * kTargetExperts;
  const bool drafter = id >= target_ids;
  const uint32_t group = drafter ? (id - target_ids) / kDrafterExperts : id / kTargetExperts;
  const uint32_t expert = drafter ? (id - target_ids) % kDrafterExperts : id % kTargetExperts;
  return std::string(drafter ? "mtp." : "layers.") + std::to_string(group) + ".ffn.experts." +
         std::to_string(expert) + "." + kField[field];
}

// An extent serves a view when the view's destination lies within the bytes
// the extent must deliver and the file position it maps the view to is the
// tensor's own place: same file, same file size, same offset.
inline bool extent_serves(const RecordExtent &e, const RecordView &v, const CkptTensor &t) {
  if (e.path != t.path || e.expected_file_bytes != t.file_bytes) return false;
  if (!range_within(Range{e.dst_offset, e.need()}, Range{v.offset, v.bytes})) return false;
  return e.file_offset + (v.offset - e.dst_offset) == t.offset;
}

// The engine's checks before any read (engine/src/forward.cu:1781-1832): per
// record, each extent's required bytes fit the extent and its file, the buffer
// geometry holds, the id is a valid expert seen once; then every view has its
// tensor's byte count and is served by some extent, and every extent serves
// some view.
inline void validate_records(const std::vector<ExpertRecord> &records,
                             const std::map<std::string, CkptTensor> &ckpt) {
  std::vector<bool> seen(kExpertIds, false);
  for (const auto &r : records) {
    for (const auto &e : r.extents) {
      if (e.need() > e.bytes || !range_within(Range{0, e.expected_file_bytes}, Range{e.file_offset, e.need()}))
        throw RecordError("expert extent's required bytes exceed the extent or run past its file");
    }
    check_destinations(r);
    if (r.id >= kExpertIds || seen[r.id]) throw RecordError("expert id out of range or listed twice");
    seen[r.id] = true;
    std::vector<bool> serving(r.extents.size(), false);
    for (int f = 0; f < 6; ++f) {
      const std::string name = expert_tensor_name(r.id, f);
      const auto it = ckpt.find(name);
      if (it == ckpt.end()) throw RecordError("the checkpoint has no tensor " + name);
      const CkptTensor &t = it->second;
      if (r.view[f].bytes != t.bytes) throw RecordError("record view size differs from tensor " + name);
      bool served = false;
      for (size_t k = 0; k < r.extents.size(); ++k)
        if (extent_serves(r.extents[k], r.view[f], t)) served = serving[k] = true;
      if (!served) throw RecordError("no extent reads tensor " + name + " from its place in the checkpoint");
    }
    if (std::find(serving.begin(), serving.end(), false) != serving.end())
      throw RecordError("expert record has an extent that reads none of its tensors");
  }
}

// Reads a record's extents into dst (record.bytes bytes). An extent may end at
// EOF before `bytes` (its file is shorter than the aligned read) as long as its
// required bytes arrived; the rest of the extent is zeroed.
inline void read_record(const ExpertRecord &r, uint8_t *dst) {
  for (const auto &e : r.extents) {
    Fd fd(e.path);
    if (fd.size() != e.expected_file_bytes) throw RecordError("expert file size changed: " + e.path);
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
