// mx_npue.cpp -- the .npue weight container, read for the GPU backend.
//
// Format (runtime/include/runtime/model.hpp; writer tools/lib/npue.py:790-870,
// reader runtime/src/model.cpp:214-380):
//   [0, 64)                      header: "NPUE", version 1, arch, flags,
//                                json_offset, json_length, data_offset (4096-
//                                aligned), data_length, 16 reserved bytes
//   [json_offset, +json_length)  UTF-8 JSON {"config": {...}, "tensors": [...]}
//   [data_offset, +data_length)  tensor bytes; a tensor's "offset" is relative
//                                to data_offset
// The file is mapped read-only and tensors are handed out as pointers into the
// mapping, as the reference does; nothing is copied at open.
//
// The directory is parsed by a small JSON reader of this file's own that
// accepts what json.dumps writes (objects, arrays, strings with every JSON
// escape including \uXXXX surrogate pairs, numbers, true/false/null) and
// refuses anything else by name. Config values keep the reference's
// convention: a string value is its unescaped text, a number or literal its
// JSON text, and an object or array its raw JSON text.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "mx_host.hpp"

namespace {

struct HeaderBytes {
  char magic[4];
  uint32_t version, arch, flags;
  uint64_t json_offset, json_length, data_offset, data_length;
  uint8_t reserved[16];
} __attribute__((packed));
static_assert(sizeof(HeaderBytes) == 64, "the .npue header is 64 bytes");

struct TensorRec {
  std::string name, role, dtype, layout_kind, layout_hash;
  std::vector<int64_t> logical, padded;
  uint64_t offset = 0, nbytes = 0;
  int64_t tile_k = 0, tile_n = 0, mac_s = 0, mac_t = 0;
  bool has_layout = false;
};

// Recursive-descent reader over the directory text. Every method advances
// `i` past what it consumed; errors carry the byte position. Objects and
// arrays nest at most kMaxDepth deep (the packer writes four levels), so a
// crafted directory cannot exhaust the stack.
constexpr int kMaxDepth = 64;

struct Json {
  const std::string &s;
  size_t i = 0;
  int depth = 0;
  std::string err;

  explicit Json(const std::string &text) : s(text) {}

  bool fail(const std::string &what) {
    if (err.empty()) err = "directory byte " + std::to_string(i) + ": " + what;
    return false;
  }
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
  }
  bool peek(char c) {
    ws();
    return i < s.size() && s[i] == c;
  }
  bool eat(char c) {
    if (!peek(c)) return fail(std::string("expected '") + c + "'");
    ++i;
    return true;
  }
  static void utf8(uint32_t cp, std::string &out) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t &v) {
    if (i + 4 > s.size()) return fail("truncated \\u escape");
    v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s[i++];
      uint32_t d;
      if (c >= '0' && c <= '9') d = static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') d = static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') d = static_cast<uint32_t>(c - 'A' + 10);
      else return fail(std::string("'") + c + "' in a \\u escape");
      v = v * 16 + d;
    }
    return true;
  }
  bool string(std::string &out) {
    out.clear();
    if (!eat('"')) return false;
    while (true) {
      if (i >= s.size()) return fail("unterminated string");
      const char c = s[i++];
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20) return fail("control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i >= s.size()) return fail("unterminated escape");
      const char e = s[i++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            uint32_t lo;
            if (i + 2 > s.size() || s[i] != '\\' || s[i + 1] != 'u')
              return fail("unpaired surrogate in a \\u escape");
            i += 2;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("bad low surrogate in a \\u escape");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("lone low surrogate in a \\u escape");
          }
          utf8(cp, out);
          break;
        }
        default:
          return fail(std::string("unknown escape '\\") + e + "'");
      }
    }
  }
  // A number or true/false/null, returned as its text.
  bool scalar(std::string &out) {
    ws();
    const size_t b = i;
    if (s.compare(i, 4, "true") == 0) i += 4;
    else if (s.compare(i, 5, "false") == 0) i += 5;
    else if (s.compare(i, 4, "null") == 0) i += 4;
    else {
      if (i < s.size() && s[i] == '-') ++i;
      const size_t d0 = i;
      while (i < s.size() && ((s[i] >= '0' && s[i] <= '9') || s[i] == '.' || s[i] == 'e' ||
                              s[i] == 'E' || s[i] == '+' || s[i] == '-'))
        ++i;
      if (i == d0) return fail("expected a value");
    }
    out = s.substr(b, i - b);
    return true;
  }
  // Any value, skipped; `raw` (if given) receives its exact text.
  bool value(std::string *raw = nullptr) {
    ws();
    const size_t b = i;
    if (i >= s.size()) return fail("expected a value");
    std::string tmp;
    if ((s[i] == '{' || s[i] == '[') && depth >= kMaxDepth)
      return fail("objects and arrays nested deeper than " + std::to_string(kMaxDepth));
    if (s[i] == '"') {
      if (!string(tmp)) return false;
    } else if (s[i] == '{') {
      ++i;
      ++depth;
      if (!peek('}')) {
        do {
          if (!string(tmp) || !eat(':') || !value()) return false;
        } while (peek(',') && (++i, true));
      }
      if (!eat('}')) return false;
      --depth;
    } else if (s[i] == '[') {
      ++i;
      ++depth;
      if (!peek(']')) {
        do {
          if (!value()) return false;
        } while (peek(',') && (++i, true));
      }
      if (!eat(']')) return false;
      --depth;
    } else if (!scalar(tmp)) {
      return false;
    }
    if (raw) *raw = s.substr(b, i - b);
    return true;
  }
  bool integer(int64_t &v) {
    std::string t;
    if (!scalar(t)) return false;
    char *end = nullptr;
    v = std::strtoll(t.c_str(), &end, 10);
    if (t.empty() || *end) return fail("'" + t + "' is not an integer");
    return true;
  }
  bool int_array(std::vector<int64_t> &out) {
    out.clear();
    if (!eat('[')) return false;
    if (!peek(']')) {
      do {
        int64_t v;
        if (!integer(v)) return false;
        out.push_back(v);
      } while (peek(',') && (++i, true));
    }
    return eat(']');
  }
};

}  // namespace

struct mx_npue {
  std::string path;
  const uint8_t *base = nullptr;
  size_t size = 0;
  uint32_t version = 0, arch = 0, flags = 0;
  uint64_t data_offset = 0, data_length = 0;
  std::map<std::string, std::string> config;
  std::map<std::string, TensorRec> tensors;
  std::vector<std::string> order;  // tensor names in directory order
};

namespace {

using mx::fail;

int parse_layout(Json &j, TensorRec &t) {
  if (!j.eat('{')) return -1;
  t.has_layout = true;
  if (!j.peek('}')) {
    do {
      std::string k, v;
      if (!j.string(k) || !j.eat(':')) return -1;
      bool ok = true;
      if (k == "kind") ok = j.peek('"') ? j.string(t.layout_kind) : j.value();
      else if (k == "tile_k") ok = j.integer(t.tile_k);
      else if (k == "tile_n") ok = j.integer(t.tile_n);
      else if (k == "mac_s") ok = j.integer(t.mac_s);
      else if (k == "mac_t") ok = j.integer(t.mac_t);
      else ok = j.value();
      if (!ok) return -1;
    } while (j.peek(',') && (++j.i, true));
  }
  return j.eat('}') ? 0 : -1;
}

int parse_directory(mx_npue *f, const std::string &js) {
  Json j(js);
  auto bad = [&]() { return fail(MX_E_INVALID, f->path + ": .npue " + j.err); };
  if (!j.eat('{')) return bad();
  if (!j.peek('}')) {
    do {
      std::string key;
      if (!j.string(key) || !j.eat(':')) return bad();
      if (key == "config") {
        if (!j.eat('{')) return bad();
        if (!j.peek('}')) {
          do {
            std::string ck, cv;
            if (!j.string(ck) || !j.eat(':')) return bad();
            if (j.peek('"')) {
              if (!j.string(cv)) return bad();
            } else if (j.peek('{') || j.peek('[')) {
              if (!j.value(&cv)) return bad();
            } else if (!j.scalar(cv)) {
              return bad();
            }
            f->config[ck] = cv;
          } while (j.peek(',') && (++j.i, true));
        }
        if (!j.eat('}')) return bad();
      } else if (key == "tensors") {
        if (!j.eat('[')) return bad();
        if (!j.peek(']')) {
          do {
            TensorRec t;
            if (!j.eat('{')) return bad();
            if (!j.peek('}')) {
              do {
                std::string tk;
                if (!j.string(tk) || !j.eat(':')) return bad();
                bool ok = true;
                int64_t v = 0;
                if (tk == "name") ok = j.string(t.name);
                else if (tk == "role") ok = j.string(t.role);
                else if (tk == "dtype") ok = j.string(t.dtype);
                else if (tk == "layout_hash") ok = j.string(t.layout_hash);
                else if (tk == "logical_shape") ok = j.int_array(t.logical);
                else if (tk == "padded_shape") ok = j.int_array(t.padded);
                else if (tk == "offset") {
                  ok = j.integer(v);
                  t.offset = static_cast<uint64_t>(v);
                  if (ok && v < 0) return fail(MX_E_INVALID, f->path + ": negative tensor offset");
                } else if (tk == "nbytes") {
                  ok = j.integer(v);
                  t.nbytes = static_cast<uint64_t>(v);
                  if (ok && v < 0) return fail(MX_E_INVALID, f->path + ": negative tensor size");
                } else if (tk == "layout") {
                  ok = parse_layout(j, t) == 0;
                } else {
                  ok = j.value();
                }
                if (!ok) return bad();
              } while (j.peek(',') && (++j.i, true));
            }
            if (!j.eat('}')) return bad();
            if (t.name.empty()) return fail(MX_E_INVALID, f->path + ": a tensor has no name");
            if (t.offset > f->data_length || t.nbytes > f->data_length - t.offset)
              return fail(MX_E_INVALID, f->path + ": tensor " + t.name +
                                            " runs past the data segment");
            if (f->tensors.count(t.name))
              return fail(MX_E_INVALID, f->path + ": tensor " + t.name + " is listed twice");
            f->order.push_back(t.name);
            f->tensors[t.name] = t;
          } while (j.peek(',') && (++j.i, true));
        }
        if (!j.eat(']')) return bad();
      } else if (!j.value()) {
        return bad();
      }
    } while (j.peek(',') && (++j.i, true));
  }
  if (!j.eat('}')) return bad();
  return MX_OK;
}

}  // namespace

namespace mx {

const TensorRecView npue_tensor(const mx_npue *f, const std::string &name) {
  TensorRecView v{};
  auto it = f->tensors.find(name);
  if (it == f->tensors.end()) return v;
  const TensorRec &t = it->second;
  v.found = true;
  v.dtype = t.dtype;
  v.padded = t.padded;
  v.logical = t.logical;
  v.block_panel = t.has_layout && t.layout_kind == "block_panel";
  v.has_layout = t.has_layout;
  v.tile_k = t.tile_k;
  v.tile_n = t.tile_n;
  v.mac_s = t.mac_s;
  v.mac_t = t.mac_t;
  v.data = f->base + f->data_offset + t.offset;
  v.nbytes = t.nbytes;
  return v;
}

bool npue_config(const mx_npue *f, const std::string &key, std::string &out) {
  auto it = f->config.find(key);
  if (it == f->config.end()) return false;
  out = it->second;
  return true;
}

}  // namespace mx

extern "C" {

int mx_npue_open(const char *path, mx_npue **out) {
  mx::clear_error();
  if (!path || !out) return fail(MX_E_INVALID, "npue_open: null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(MX_E_INVALID, std::string("cannot open ") + path);
  struct stat st {};
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    return fail(MX_E_INVALID, std::string("cannot stat ") + path);
  }
  const size_t size = static_cast<size_t>(st.st_size);
  if (size < sizeof(HeaderBytes)) {
    ::close(fd);
    return fail(MX_E_INVALID, std::string(path) + ": truncated (" + std::to_string(size) +
                                  " bytes, the header alone is 64)");
  }
  void *m = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return fail(MX_E_INVALID, std::string("cannot map ") + path);
  mx_npue *f = new mx_npue;
  f->path = path;
  f->base = static_cast<const uint8_t *>(m);
  f->size = size;
  HeaderBytes h;
  std::memcpy(&h, f->base, sizeof h);
  auto refuse = [&](const std::string &why) {
    mx_npue_close(f);
    return fail(MX_E_INVALID, std::string(path) + ": " + why);
  };
  if (std::memcmp(h.magic, "NPUE", 4) != 0) return refuse("not a .npue file (magic)");
  if (h.version != 1) return refuse("version " + std::to_string(h.version) + ", expected 1");
  if (h.data_offset % 4096 != 0) return refuse("data_offset is not 4096-aligned");
  if (h.data_offset > size || h.data_length != size - h.data_offset)
    return refuse("file size does not match the header's data segment");
  if (h.json_offset > size || h.json_length > size - h.json_offset ||
      h.json_offset + h.json_length > h.data_offset)
    return refuse("the directory lies outside the file or overlaps the data");
  f->version = h.version;
  f->arch = h.arch;
  f->flags = h.flags;
  f->data_offset = h.data_offset;
  f->data_length = h.data_length;
  const std::string js(reinterpret_cast<const char *>(f->base + h.json_offset), h.json_length);
  const int rc = parse_directory(f, js);
  if (rc) {
    mx_npue_close(f);
    return rc;
  }
  *out = f;
  return MX_OK;
}

void mx_npue_close(mx_npue *f) {
  if (!f) return;
  if (f->base) ::munmap(const_cast<uint8_t *>(f->base), f->size);
  delete f;
}

int mx_npue_config(const mx_npue *f, const char *key, char *buf, size_t len) {
  mx::clear_error();
  if (!f || !key) return fail(MX_E_INVALID, "npue_config: null argument");
  std::string v;
  if (!mx::npue_config(f, key, v))
    return fail(MX_E_INVALID, f->path + ": no config key " + key);
  if (buf && len) {
    const size_t n = v.size() < len - 1 ? v.size() : len - 1;
    std::memcpy(buf, v.data(), n);
    buf[n] = 0;
  }
  return static_cast<int>(v.size());
}

int mx_npue_tensor_count(const mx_npue *f) {
  return f ? static_cast<int>(f->order.size()) : -1;
}

const char *mx_npue_tensor_name(const mx_npue *f, int index) {
  if (!f || index < 0 || index >= static_cast<int>(f->order.size())) return nullptr;
  return f->order[static_cast<size_t>(index)].c_str();
}

int mx_npue_tensor(const mx_npue *f, const char *name, mx_npue_tensor_info *out) {
  mx::clear_error();
  if (!f || !name || !out) return fail(MX_E_INVALID, "npue_tensor: null argument");
  const mx::TensorRecView v = mx::npue_tensor(f, name);
  if (!v.found) return fail(MX_E_INVALID, f->path + ": no tensor named " + name);
  std::memset(out, 0, sizeof *out);
  std::strncpy(out->dtype, v.dtype.c_str(), sizeof out->dtype - 1);
  out->ndim = static_cast<int>(v.padded.size() < 4 ? v.padded.size() : 4);
  for (int d = 0; d < out->ndim; ++d) out->padded_shape[d] = v.padded[static_cast<size_t>(d)];
  const int nl = static_cast<int>(v.logical.size() < 4 ? v.logical.size() : 4);
  for (int d = 0; d < nl; ++d) out->logical_shape[d] = v.logical[static_cast<size_t>(d)];
  out->block_panel = v.block_panel ? 1 : 0;
  out->tile_k = v.tile_k;
  out->tile_n = v.tile_n;
  out->mac_s = v.mac_s;
  out->mac_t = v.mac_t;
  out->data = v.data;
  out->nbytes = v.nbytes;
  return MX_OK;
}

}  // extern "C"
