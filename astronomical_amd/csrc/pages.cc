// Expert pages from safetensors checkpoints: header parsing, the startup-validated layer plan,
// the selected-page manifest and the bounded reader that writes exactly the selected experts'
// bytes into host or HIP device buffers.  Host code only (no kernel): it builds with the host
// compiler, which is also how the sanitizer build of the host library takes it.
//
// Follows the reference's expert paging:
//   parse_safetensors_header           expert_paging/safetensors_header.rs:171-276
//   read_bounded_safetensors_json_header safetensors/header.rs:109-158
//   build_quantized_expert_layer_plan  qwen3_5_moe/expert_paging/quantized_expert_layer_plan.rs:29-330
//   validate_expert_ids / validate_quantization_contract / validate_source_intervals
//                                      expert_paging/quantized_expert_validation.rs:9-140
//   build_source_manifests / contiguous_selected_runs  expert_paging/source_manifests.rs:9-99
//   build_page_slot_by_global_expert_id expert_paging/quantized_expert_manifest.rs:420-451
//   load_quantized_expert_page         expert_paging/bounded_expert_reader.rs:35-117
//   resident gate/up fusion plan and concatenation
//                                      qwen3_5_moe/expert_residency/resident_gate_up_fusion.rs:109-268
#include <hip/hip_runtime_api.h>

#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/astro_moe.h"
#include "status.h"

using astro::report;
using astro::report_ok;

namespace {

const char *const kHeaderOp = "parse a safetensors header";
const char *const kPlanOp = "build a quantized expert layer plan";
const char *const kPageOp = "build a quantized expert page manifest";
const char *const kLoadOp = "load a quantized expert page";

constexpr uint64_t kMaxHeaderBytes = 64ull << 20;  // safetensors_header.rs:19

// ------------------------------------------------------------------ JSON (the header's subset)

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool boolean = false;
  bool integral = false;  // a number without fraction or exponent that fits int64
  int64_t integer = 0;
  std::string text;       // string value, or the number's spelling
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json *get(const char *key) const {
    for (const auto &m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

// The JSON the reference's serde_json reading accepts (serde_json 1.0.151 from_slice through
// strict_json.rs:11-110): RFC 8259 with strings of valid UTF-8 (no raw control characters, no
// lone surrogate escapes), numbers that are finite as f64, at most kMaxJsonNesting nested
// arrays and objects (serde_json's recursion limit of 128), and no duplicate key in any object.
// An integer literal is integral when it fits int64 (serde_json's as_i64); "-0" is not (serde_json
// reads it as the float -0.0).
constexpr int kMaxJsonNesting = 127;

class JsonParser {
 public:
  JsonParser(const char *p, size_t n) : p_(p), end_(p + n) {}

  // whole document: one value, then only whitespace
  bool document(Json &out) {
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  const char *p_, *end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char *s) {
    const size_t n = strlen(s);
    if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(std::string &s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xc0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3f));
    } else if (c < 0x10000) {
      s += (char)(0xe0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3f));
      s += (char)(0x80 | (c & 0x3f));
    } else {
      s += (char)(0xf0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3f));
      s += (char)(0x80 | ((c >> 6) & 0x3f));
      s += (char)(0x80 | (c & 0x3f));
    }
  }
  bool hex4(uint32_t &v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string &s) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_) {
      const unsigned char c = (unsigned char)*p_++;
      if (c == '"') return true;
      if (c < 0x20) return false;
      if (c >= 0x80) {  // one UTF-8 sequence, validated (no overlong form, surrogate or > U+10FFFF)
        const int n = c >= 0xf0 ? 3 : c >= 0xe0 ? 2 : c >= 0xc2 ? 1 : -1;
        if (n < 0 || c > 0xf4 || end_ - p_ < n) return false;
        const unsigned char c1 = (unsigned char)p_[0];
        if ((c1 & 0xc0) != 0x80) return false;
        if (c == 0xe0 && c1 < 0xa0) return false;  // overlong 3-byte
        if (c == 0xed && c1 >= 0xa0) return false;  // UTF-16 surrogate
        if (c == 0xf0 && c1 < 0x90) return false;  // overlong 4-byte
        if (c == 0xf4 && c1 >= 0x90) return false;  // above U+10FFFF
        for (int i = 1; i < n; ++i)
          if (((unsigned char)p_[i] & 0xc0) != 0x80) return false;
        s += (char)c;
        s.append(p_, (size_t)n);
        p_ += n;
        continue;
      }
      if (c != '\\') {
        s += (char)c;
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(c1)) return false;
          if (c1 >= 0xd800 && c1 < 0xdc00) {  // surrogate pair
            uint32_t c2;
            if (!lit("\\u") || !hex4(c2) || c2 < 0xdc00 || c2 >= 0xe000) return false;
            c1 = 0x10000 + ((c1 - 0xd800) << 10) + (c2 - 0xdc00);
          } else if (c1 >= 0xdc00 && c1 < 0xe000) {
            return false;
          }
          utf8(s, c1);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool number(Json &out) {
    const char *b = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_) return false;
    if (*p_ == '0') {
      ++p_;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    } else {
      return false;
    }
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    out.kind = Json::Number;
    out.text.assign(b, p_);
    if (integral && out.text != "-0") {
      errno = 0;
      char *e = nullptr;
      const long long v = strtoll(out.text.c_str(), &e, 10);
      if (errno == 0 && e && *e == 0) {
        out.integral = true;
        out.integer = v;
      }
    }
    // a literal past f64's range is an error (an integer of any size still reads as a float)
    if (!out.integral && std::isinf(strtod(out.text.c_str(), nullptr))) return false;
    return true;
  }
  // depth: the arrays and objects this value is nested in
  bool value(Json &out, int depth) {
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if ((c == '{' || c == '[') && depth >= kMaxJsonNesting) return false;
    if (c == '{') {
      ++p_;
      out.kind = Json::Object;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      std::set<std::string> keys;
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        if (!keys.insert(key).second) return false;  // duplicate entry
        ws();
        if (p_ >= end_ || *p_ != ':') return false;
        ++p_;
        Json v;
        if (!value(v, depth + 1)) return false;
        out.members.emplace_back(std::move(key), std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      out.kind = Json::Array;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        Json v;
        if (!value(v, depth + 1)) return false;
        out.items.push_back(std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      out.kind = Json::String;
      return string(out.text);
    }
    if (lit("true")) {
      out.kind = Json::Bool;
      out.boolean = true;
      return true;
    }
    if (lit("false")) {
      out.kind = Json::Bool;
      return true;
    }
    if (lit("null")) return true;
    return number(out);
  }
};

// compact JSON spelling of a value, for messages that quote it
std::string json_text(const Json &v) {
  switch (v.kind) {
    case Json::Null: return "null";
    case Json::Bool: return v.boolean ? "true" : "false";
    case Json::Number: return v.text;
    case Json::String: return "\"" + v.text + "\"";
    case Json::Array: {
      std::string s = "[";
      for (size_t i = 0; i < v.items.size(); ++i) s += (i ? "," : "") + json_text(v.items[i]);
      return s + "]";
    }
    case Json::Object: {
      std::string s = "{";
      for (size_t i = 0; i < v.members.size(); ++i)
        s += (i ? ",\"" : "\"") + v.members[i].first + "\":" + json_text(v.members[i].second);
      return s + "}";
    }
  }
  return "";
}

// ------------------------------------------------------------------ safetensors headers

const char *const kDtypeNames[] = {"BOOL", "I8", "U8", "F8_E4M3", "F8_E5M2", "I16", "U16",
                                   "F16", "BF16", "I32", "U32", "F32", "I64", "U64"};
const int kDtypeWidths[] = {1, 1, 1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8};
constexpr int kNumDtypes = 14;

int dtype_of(const std::string &s) {
  for (int i = 0; i < kNumDtypes; ++i)
    if (s == kDtypeNames[i]) return i;
  return -1;
}

struct TensorEntry {
  int dtype;
  std::vector<int64_t> shape;
  uint64_t start, end;  // file-relative
};

struct Header {
  std::map<std::string, TensorEntry> tensors;
  uint64_t payload_start = 0, file_size = 0;
};

bool read_exact(int fd, void *dst, uint64_t n, uint64_t off) {
  char *p = (char *)dst;
  while (n > 0) {
    const ssize_t r = pread(fd, p, n > (1u << 30) ? (1u << 30) : (size_t)n, (off_t)off);
    if (r < 0) {
      if (errno == EINTR) continue;
      return false;
    }
    if (r == 0) {
      errno = 0;  // the file ended before the requested bytes
      return false;
    }
    p += r;
    n -= (uint64_t)r;
    off += (uint64_t)r;
  }
  return true;
}

// parse_safetensors_header (safetensors_header.rs:171-276): 0 or a status with the message set
int parse_header(const std::string &path, Header &h) {
  struct stat st;
  if (stat(path.c_str(), &st) != 0) {
    if (errno == ENOENT) return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "safetensors file does not exist: \"%s\"", path.c_str());
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "I/O error reading safetensors file: %s", strerror(errno));
  }
  if (!S_ISREG(st.st_mode))
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "safetensors path is not a regular file: \"%s\"", path.c_str());
  const uint64_t size = (uint64_t)st.st_size;
  if (size < 8)
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp,
                  "safetensors file is too small to contain a header length prefix: %llu bytes",
                  (unsigned long long)size);
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "I/O error reading safetensors file: %s", strerror(errno));
  unsigned char pre[8];
  if (!read_exact(fd, pre, 8, 0)) {
    close(fd);
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "I/O error reading safetensors file: %s",
                  errno ? strerror(errno) : "safetensors file ended before the requested bytes");
  }
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | pre[i];
  if (n > kMaxHeaderBytes) {
    close(fd);
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp,
                  "safetensors header length %llu exceeds the safety limit of %llu bytes",
                  (unsigned long long)n, (unsigned long long)kMaxHeaderBytes);
  }
  if (8 + n > size) {
    close(fd);
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp,
                  "safetensors header extends beyond the file: header ends at %llu but file is %llu bytes",
                  (unsigned long long)(8 + n), (unsigned long long)size);
  }
  std::vector<char> text(n);
  const bool got = read_exact(fd, text.data(), n, 8);
  close(fd);
  if (!got)
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "I/O error reading safetensors file: %s",
                  errno ? strerror(errno) : "safetensors file ended before the requested bytes");
  Json doc;
  JsonParser parser(text.data(), text.size());
  if (!parser.document(doc) || doc.kind != Json::Object)
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "safetensors header must contain valid JSON");
  h = Header();
  h.payload_start = 8 + n;
  h.file_size = size;
  const uint64_t payload = size - h.payload_start;
  // entries in key order (byte-wise), as the reference's map of them iterates: with several bad
  // entries, the first by name is the one reported
  std::vector<const std::pair<std::string, Json> *> entries;
  for (const auto &m : doc.members) entries.push_back(&m);
  std::sort(entries.begin(), entries.end(), [](const auto *x, const auto *y) { return x->first < y->first; });
  for (const auto *m : entries) {
    const std::string &name = m->first;
    if (name == "__metadata__") continue;
    const Json &t = m->second;
    if (t.kind != Json::Object)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "safetensors header must be a JSON object, got %s",
                    json_text(t).c_str());
    const Json *dt = t.get("dtype");
    if (!dt || dt->kind != Json::String)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" has an unsupported dtype: \"missing\"", name.c_str());
    const int dtype = dtype_of(dt->text);
    if (dtype < 0)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" has an unsupported dtype: \"%s\"", name.c_str(),
                    dt->text.c_str());
    const Json *sh = t.get("shape");
    if (!sh || sh->kind != Json::Array)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" has an invalid shape", name.c_str());
    TensorEntry e;
    e.dtype = dtype;
    for (const Json &d : sh->items) {
      if (d.kind != Json::Number || !d.integral || d.integer < 0)
        return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" has an invalid shape", name.c_str());
      e.shape.push_back(d.integer);
    }
    const Json *off = t.get("data_offsets");
    if (!off || off->kind != Json::Array || off->items.size() != 2 || off->items[0].kind != Json::Number ||
        off->items[1].kind != Json::Number || !off->items[0].integral || !off->items[1].integral ||
        off->items[0].integer < 0 || off->items[1].integer < off->items[0].integer)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" has invalid data_offsets", name.c_str());
    const uint64_t s = (uint64_t)off->items[0].integer, en = (uint64_t)off->items[1].integer;
    if (en > payload)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp,
                    "tensor \"%s\" data_offsets are outside the file payload: [%llu, %llu) vs payload size %llu",
                    name.c_str(), (unsigned long long)s, (unsigned long long)en, (unsigned long long)payload);
    // element count with checked 64-bit products; an overflow reports 0 expected bytes
    uint64_t count = 1;
    bool overflow = false;
    for (int64_t d : e.shape)
      if (!overflow && __builtin_mul_overflow(count, (uint64_t)d, &count)) overflow = true;
    const uint64_t expect = overflow ? 0 : count * (uint64_t)kDtypeWidths[dtype];
    if (overflow || expect != en - s)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp,
                    "tensor \"%s\" byte count mismatch: header declares %llu bytes but shape\xc3\x97"
                    "dtype expects %llu bytes",
                    name.c_str(), (unsigned long long)(en - s), (unsigned long long)expect);
    e.start = h.payload_start + s;
    e.end = h.payload_start + en;
    h.tensors[name] = e;
  }
  return ASTRO_MOE_OK;
}

// ------------------------------------------------------------------ layer plan

const char *const kProjections[3] = {"gate_proj", "up_proj", "down_proj"};
const char *const kParameters[3] = {"weight", "scales", "biases"};

// validate_quantization_contract (quantized_expert_validation.rs:37-62)
int check_contract(const char *op, int bits, int group) {
  if (bits <= 0) return report(ASTRO_MOE_INVALID_ARGUMENT, op, "quantization bits must be a positive integer");
  if (group <= 0) return report(ASTRO_MOE_INVALID_ARGUMENT, op, "quantization group_size must be a positive integer");
  if (((int64_t)group * bits) % 32 != 0)
    return report(ASTRO_MOE_INVALID_ARGUMENT, op,
                  "quantized expert groups must pack into whole U32 elements: bits=%d, group_size=%d", bits, group);
  return ASTRO_MOE_OK;
}

std::string join_path(const std::string &dir, const std::string &file) {
  if (dir.empty() || (!file.empty() && file[0] == '/')) return file;
  return dir.back() == '/' ? dir + file : dir + "/" + file;
}

// validate_expert_ids (quantized_expert_validation.rs:9-35), ids as int32
int check_ids(const int32_t *ids, int32_t n, int32_t capacity) {
  if (n <= 0 || !ids) return report(ASTRO_MOE_INVALID_ARGUMENT, kPageOp, "quantized expert page must select at least one expert");
  for (int32_t i = 0; i < n; ++i)
    if (ids[i] < 0) return report(ASTRO_MOE_INVALID_ARGUMENT, kPageOp, "expert IDs must be non-negative integers");
  int32_t mx = 0;
  for (int32_t i = 0; i < n; ++i) mx = std::max(mx, ids[i]);
  if (mx >= capacity)
    return report(ASTRO_MOE_INVALID_ARGUMENT, kPageOp,
                  "selected expert IDs exceed the quantized layer's expert capacity: max %d, got %d", capacity, mx);
  for (int32_t i = 1; i < n; ++i)
    if (ids[i - 1] >= ids[i])
      return report(ASTRO_MOE_INVALID_ARGUMENT, kPageOp, "expert IDs must be unique and strictly ascending");
  return ASTRO_MOE_OK;
}

struct Run {
  int32_t start, count, first_slot;
};

// contiguous_selected_runs (source_manifests.rs:77-99): runs of consecutive ids with the
// page slot of their first id
std::vector<Run> selected_runs(const int32_t *ids, int32_t n) {
  std::vector<Run> runs;
  int32_t i = 0;
  while (i < n) {
    int32_t j = i + 1;
    while (j < n && ids[j] == ids[j - 1] + 1) ++j;
    runs.push_back({ids[i], j - i, i});
    i = j;
  }
  return runs;
}

// every read of the page, in (projection, parameter, run) order
std::vector<astro_moe_page_interval> page_intervals(const astro_moe_expert_layer_plan &plan,
                                                    const int32_t *ids, int32_t n) {
  const std::vector<Run> runs = selected_runs(ids, n);
  std::vector<astro_moe_page_interval> out;
  for (int p = 0; p < 3; ++p)
    for (int q = 0; q < 3; ++q) {
      const astro_moe_tensor_source &s = plan.src[p][q];
      for (const Run &r : runs) {
        astro_moe_page_interval iv{};
        iv.projection = p;
        iv.parameter = q;
        iv.expert_start = r.start;
        iv.expert_count = r.count;
        iv.first_page_slot = r.first_slot;
        iv.file_offset = s.file_offset + (uint64_t)r.start * s.bytes_per_expert;
        iv.byte_count = (uint64_t)r.count * s.bytes_per_expert;
        iv.virtual_offset = (uint64_t)r.first_slot * s.bytes_per_expert;
        out.push_back(iv);
      }
    }
  return out;
}

int check_plan(const astro_moe_expert_layer_plan *plan, const char *op) {
  if (!plan) return report(ASTRO_MOE_INVALID_ARGUMENT, op, "layer plan must be non-null");
  if (plan->expert_capacity <= 0) return report(ASTRO_MOE_INVALID_ARGUMENT, op, "layer plan has no experts");
  return ASTRO_MOE_OK;
}

// ------------------------------------------------------------------ bounded reads

struct FileSet {
  std::map<std::string, int> fds;
  ~FileSet() {
    for (auto &f : fds) close(f.second);
  }
  int get(const std::string &path) {
    auto it = fds.find(path);
    if (it != fds.end()) return it->second;
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd >= 0) fds[path] = fd;
    return fd;
  }
};

// One block copy of the page: `bytes` from file offset `off` to destination offset `dst_off`
// of buffer (p, q).
struct Copy {
  int p, q;
  uint64_t off, bytes, dst_off;
};

}  // namespace

extern "C" {

int astro_moe_safetensors_tensor(const char *path, const char *tensor_name, int32_t *dtype,
                                 int32_t *rank, int64_t *shape, uint64_t *file_offset,
                                 uint64_t *byte_count) {
  if (!path || !tensor_name) return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "path and tensor name must be non-null");
  Header h;
  const int rc = parse_header(path, h);
  if (rc) return rc;
  auto it = h.tensors.find(tensor_name);
  if (it == h.tensors.end())
    return report(ASTRO_MOE_INVALID_ARGUMENT, kHeaderOp, "tensor \"%s\" is not in the safetensors header", tensor_name);
  const TensorEntry &e = it->second;
  if (dtype) *dtype = e.dtype;
  if (rank) *rank = (int32_t)e.shape.size();
  if (shape)
    for (size_t i = 0; i < e.shape.size() && i < 8; ++i) shape[i] = e.shape[i];
  if (file_offset) *file_offset = e.start;
  if (byte_count) *byte_count = e.end - e.start;
  return report_ok();
}

int astro_moe_build_expert_layer_plan(const char *model_dir, const char *const *map_tensor_names,
                                const char *const *map_shard_files, int32_t map_len,
                                const char *layer_prefix, const int32_t bits[3],
                                const int32_t group_size[3], astro_moe_expert_layer_plan *plan) {
  if (!plan || !layer_prefix || !bits || !group_size || map_len < 0 || (map_len > 0 && (!map_tensor_names || !map_shard_files)))
    return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "plan, layer prefix, quantization profile and weight map must be non-null");
  *plan = astro_moe_expert_layer_plan{};
  const std::string dir = model_dir ? model_dir : "";
  std::map<std::string, Header> headers;  // one parse per shard
  for (int p = 0; p < 3; ++p) {
    int rc = check_contract(kPlanOp, bits[p], group_size[p]);
    if (rc) return rc;
    plan->bits[p] = bits[p];
    plan->group_size[p] = group_size[p];
    for (int q = 0; q < 3; ++q) {
      const std::string name = std::string(layer_prefix) + ".switch_mlp." + kProjections[p] + "." + kParameters[q];
      const char *shard = nullptr;
      for (int32_t i = 0; i < map_len; ++i)
        if (map_tensor_names[i] && map_shard_files[i] && name == map_tensor_names[i]) shard = map_shard_files[i];
      if (!shard)
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized expert page is missing index entry for tensor \"%s\"",
                      name.c_str());
      const std::string file = join_path(dir, shard);
      if (file.size() >= ASTRO_MOE_PATH_MAX)
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "shard path is longer than %d bytes", ASTRO_MOE_PATH_MAX - 1);
      auto hit = headers.find(file);
      if (hit == headers.end()) {
        Header h;
        rc = parse_header(file, h);
        if (rc) return rc;
        hit = headers.emplace(file, std::move(h)).first;
      }
      const Header &h = hit->second;
      auto te = h.tensors.find(name);
      if (te == h.tensors.end())
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized expert page is missing \"%s\" in shard header", name.c_str());
      const TensorEntry &e = te->second;
      // validate_quantized_tensor_source (quantized_expert_layer_plan.rs:219-285)
      if (q == 0 && e.dtype != ASTRO_MOE_DTYPE_U32)
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized expert tensor \"%s\" must use U32 but has %s",
                      name.c_str(), kDtypeNames[e.dtype]);
      if (q != 0 && e.dtype != ASTRO_MOE_DTYPE_F16 && e.dtype != ASTRO_MOE_DTYPE_BF16 && e.dtype != ASTRO_MOE_DTYPE_F32)
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp,
                      "quantized expert tensor \"%s\" must use float16, bfloat16, or float32 but has %s", name.c_str(),
                      kDtypeNames[e.dtype]);
      if (e.shape.size() != 3 || std::find(e.shape.begin(), e.shape.end(), 0) != e.shape.end())
        return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized expert tensor \"%s\" must have a non-empty rank-three shape",
                      name.c_str());
      astro_moe_tensor_source &s = plan->src[p][q];
      snprintf(s.source_file, sizeof s.source_file, "%s", file.c_str());
      s.dtype = e.dtype;
      for (int d = 0; d < 3; ++d) s.shape[d] = e.shape[d];
      s.file_offset = e.start;
      s.bytes_per_expert = (uint64_t)e.shape[1] * (uint64_t)e.shape[2] * (uint64_t)kDtypeWidths[e.dtype];
      s.file_size = h.file_size;
    }
    // validate_projection_quantization_geometry (quantized_expert_layer_plan.rs:287-330)
    const astro_moe_tensor_source &w = plan->src[p][0], &sc = plan->src[p][1], &bi = plan->src[p][2];
    if (memcmp(sc.shape, bi.shape, sizeof sc.shape) != 0)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized projection \"%s\" scales and biases must share a shape",
                    kProjections[p]);
    if (w.shape[0] != sc.shape[0] || w.shape[1] != sc.shape[1])
      return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized projection \"%s\" weight/scales batch dimensions differ",
                    kProjections[p]);
    const int64_t packed = sc.shape[2] * group_size[p] * bits[p] / 32;
    if (w.shape[2] != packed)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp,
                    "quantized projection \"%s\" has an invalid packed weight width: expected %lld, got %lld",
                    kProjections[p], (long long)packed, (long long)w.shape[2]);
  }
  // one expert capacity for all nine tensors
  std::vector<int64_t> caps;
  for (int p = 0; p < 3; ++p)
    for (int q = 0; q < 3; ++q)
      if (std::find(caps.begin(), caps.end(), plan->src[p][q].shape[0]) == caps.end()) caps.push_back(plan->src[p][q].shape[0]);
  if (caps.size() != 1) {
    std::string found = "[";
    for (size_t i = 0; i < caps.size(); ++i) found += (i ? ", " : "") + std::to_string(caps[i]);
    return report(ASTRO_MOE_INVALID_ARGUMENT, kPlanOp, "quantized expert projections must share one expert capacity, found %s]",
                  found.c_str());
  }
  if (caps[0] > 0x7fffffff) return report(ASTRO_MOE_UNSUPPORTED, kPlanOp, "expert capacity exceeds the int32 range");
  plan->expert_capacity = (int32_t)caps[0];
  // the resident gate/up fusion plan (resident_gate_up_fusion.rs:119-163)
  plan->gate_up_fusable = 1;
  const char *why = nullptr;
  for (int q = 0; q < 3 && !why; ++q) {
    if (memcmp(plan->src[0][q].shape, plan->src[1][q].shape, sizeof plan->src[0][q].shape) != 0)
      why = "gate and up tensor shapes differ";
    else if (plan->src[0][q].dtype != plan->src[1][q].dtype)
      why = "gate and up tensor data types differ";
  }
  if (!why && bits[0] != bits[1]) why = "gate and up quantization bit widths differ";
  if (!why && group_size[0] != group_size[1]) why = "gate and up quantization group sizes differ";
  if (why) {
    plan->gate_up_fusable = 0;
    snprintf(plan->gate_up_separate_reason, sizeof plan->gate_up_separate_reason, "%s", why);
  }
  return report_ok();
}

int astro_moe_build_expert_page_manifest(const astro_moe_expert_layer_plan *plan, const int32_t *expert_ids,
                                   int32_t n, uint32_t *slot_of_expert, astro_moe_page_interval *intervals,
                                   int32_t max_intervals, int32_t *n_intervals, uint64_t *payload_bytes) {
  int rc = check_plan(plan, kPageOp);
  if (rc) return rc;
  rc = check_ids(expert_ids, n, plan->expert_capacity);
  if (rc) return rc;
  if (slot_of_expert) {
    // build_page_slot_by_global_expert_id (quantized_expert_manifest.rs:420-451)
    for (int32_t e = 0; e < plan->expert_capacity; ++e) slot_of_expert[e] = 0xffffffffu;
    for (int32_t i = 0; i < n; ++i) slot_of_expert[expert_ids[i]] = (uint32_t)i;
  }
  const std::vector<astro_moe_page_interval> iv = page_intervals(*plan, expert_ids, n);
  if (n_intervals) *n_intervals = (int32_t)iv.size();
  if (intervals) {
    if (max_intervals < (int32_t)iv.size())
      return report(ASTRO_MOE_INVALID_ARGUMENT, kPageOp, "interval buffer holds %d entries, the page needs %d", max_intervals,
                    (int)iv.size());
    std::copy(iv.begin(), iv.end(), intervals);
  }
  if (payload_bytes) {
    uint64_t t = 0;
    for (int p = 0; p < 3; ++p)
      for (int q = 0; q < 3; ++q) t += (uint64_t)n * plan->src[p][q].bytes_per_expert;
    *payload_bytes = t;
  }
  return report_ok();
}

int astro_moe_load_expert_page(const astro_moe_expert_layer_plan *plan, const int32_t *expert_ids,
                               int32_t n, int32_t fuse_gate_up, void *const *dst, int32_t dst_on_device,
                               void *staging, size_t staging_bytes, void *stream, uint64_t *bytes_read) {
  int rc = check_plan(plan, kLoadOp);
  if (rc) return rc;
  rc = check_ids(expert_ids, n, plan->expert_capacity);
  if (rc) return rc;
  if (fuse_gate_up && !plan->gate_up_fusable)
    return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp, "gate and up cannot be fused: %s", plan->gate_up_separate_reason);
  if (!dst) return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp, "destination buffers must be non-null");
  for (int p = 0; p < 3; ++p)
    for (int q = 0; q < 3; ++q)
      if (!(fuse_gate_up && p == 1) && !dst[p * 3 + q])
        return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp, "destination buffer %s.%s must be non-null", kProjections[p],
                      kParameters[q]);
  if (dst_on_device && staging && staging_bytes < (1u << 20))
    return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp, "the staging buffer must hold at least 1 MiB");
  // the block copies: whole runs, or, when fused, each expert's gate or up block at its place
  // in the [gate rows; up rows] row of its slot (Copy::p stays the source projection)
  std::vector<Copy> copies;
  for (const astro_moe_page_interval &iv : page_intervals(*plan, expert_ids, n)) {
    const astro_moe_tensor_source &src = plan->src[iv.projection][iv.parameter];
    if (iv.file_offset + iv.byte_count > src.file_size)
      return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp,
                    "source interval exceeds the source file: offset %llu + %llu bytes exceeds %llu bytes",
                    (unsigned long long)iv.file_offset, (unsigned long long)iv.byte_count,
                    (unsigned long long)src.file_size);
    if (!(fuse_gate_up && iv.projection < 2)) {
      copies.push_back({iv.projection, iv.parameter, iv.file_offset, iv.byte_count, iv.virtual_offset});
      continue;
    }
    const uint64_t b = src.bytes_per_expert;
    for (int32_t j = 0; j < iv.expert_count; ++j)
      copies.push_back({iv.projection, iv.parameter, iv.file_offset + (uint64_t)j * b, b,
                        ((uint64_t)(iv.first_page_slot + j) * 2 + (uint64_t)iv.projection) * b});
  }
  // file order within each shard: one forward pass over every file
  std::stable_sort(copies.begin(), copies.end(), [&](const Copy &x, const Copy &y) {
    const int c = strcmp(plan->src[x.p][x.q].source_file, plan->src[y.p][y.q].source_file);
    return c != 0 ? c < 0 : x.off < y.off;
  });
  std::vector<const char *> file_of(copies.size());
  for (size_t i = 0; i < copies.size(); ++i) file_of[i] = plan->src[copies[i].p][copies[i].q].source_file;
  FileSet files;
  uint64_t total = 0;
  auto dst_of = [&](const Copy &c) -> char * {
    const int p = fuse_gate_up && c.p < 2 ? 0 : c.p;
    return (char *)dst[p * 3 + c.q] + c.dst_off;
  };
  auto read_fail = [&](const char *path) {
    return report(ASTRO_MOE_INVALID_ARGUMENT, kLoadOp, "reader error: %s: %s", path,
                  errno ? strerror(errno) : "safetensors file ended before the requested bytes");
  };
  if (!dst_on_device) {
    for (size_t i = 0; i < copies.size(); ++i) {
      const int fd = files.get(file_of[i]);
      if (fd < 0 || !read_exact(fd, dst_of(copies[i]), copies[i].bytes, copies[i].off)) return read_fail(file_of[i]);
      total += copies[i].bytes;
    }
    if (bytes_read) *bytes_read = total;
    return report_ok();
  }
  // device: two halves of a pinned staging buffer; a half is refilled from the file once the
  // copy that last read it has completed on the stream
  hipStream_t s = (hipStream_t)stream;
  bool own = false;
  if (!staging) {
    staging_bytes = 64u << 20;
    if (hipHostMalloc(&staging, staging_bytes, hipHostMallocDefault) != hipSuccess)
      return report(ASTRO_MOE_HIP_ERROR, kLoadOp, "could not allocate %zu bytes of pinned staging memory", staging_bytes);
    own = true;
  }
  hipEvent_t done[2];
  bool pending[2] = {false, false};
  if (hipEventCreateWithFlags(&done[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&done[1], hipEventDisableTiming) != hipSuccess) {
    if (own) (void)hipHostFree(staging);
    return report(ASTRO_MOE_HIP_ERROR, kLoadOp, "could not create HIP events");
  }
  const size_t half = (staging_bytes / 2) & ~(size_t)4095;
  int status = ASTRO_MOE_OK;
  int cur = 0;
  for (size_t i = 0; i < copies.size() && status == ASTRO_MOE_OK; ++i) {
    const Copy &c = copies[i];
    const int fd = files.get(file_of[i]);
    if (fd < 0) {
      status = read_fail(file_of[i]);
      break;
    }
    for (uint64_t done_b = 0; done_b < c.bytes;) {
      const uint64_t chunk = std::min<uint64_t>(half, c.bytes - done_b);
      char *buf = (char *)staging + (size_t)cur * half;
      if (pending[cur] && hipEventSynchronize(done[cur]) != hipSuccess) {
        status = report(ASTRO_MOE_HIP_ERROR, kLoadOp, "staging copy failed");
        break;
      }
      pending[cur] = false;
      if (!read_exact(fd, buf, chunk, c.off + done_b)) {
        status = read_fail(file_of[i]);
        break;
      }
      if (hipMemcpyAsync(dst_of(c) + done_b, buf, chunk, hipMemcpyHostToDevice, s) != hipSuccess ||
          hipEventRecord(done[cur], s) != hipSuccess) {
        status = report(ASTRO_MOE_HIP_ERROR, kLoadOp, "host to device copy failed");
        break;
      }
      pending[cur] = true;
      cur ^= 1;
      done_b += chunk;
      total += chunk;
    }
  }
  const hipError_t se = hipStreamSynchronize(s);
  (void)hipEventDestroy(done[0]);
  (void)hipEventDestroy(done[1]);
  if (own) (void)hipHostFree(staging);
  if (status != ASTRO_MOE_OK) return status;
  if (se != hipSuccess) return report(ASTRO_MOE_HIP_ERROR, kLoadOp, "HIP error %d (%s)", (int)se, hipGetErrorString(se));
  if (bytes_read) *bytes_read = total;
  return report_ok();
}

}  // extern "C"
