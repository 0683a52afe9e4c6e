// Weight ingestion from a Hugging Face safetensors checkpoint, as the reference's loader does it
// (main.rs:160-222): keys with the `model.` prefix dropped (`^model\.` -> ""), `.A_log` read as
// `.a_log`, the language-model tensors under `language_model.`; every Linear weight transposed
// from PyTorch's [out][in] to the [in][out] layout of the reference's Burn modules
// (PyTorchToBurnAdapter); every value cast to f32 (FloatCastAdapter); the projections and the
// embedding quantised to Q8F per block of 64 by the model builder, the rest kept f32.
//
// File format: an 8-byte little-endian header length, a JSON header mapping each tensor name to
// {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the end of the header),
// then the raw little-endian tensor bytes.  The file is memory-mapped; only the tensors the
// decoder reads are touched.
#include "q35_host.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <memory>

namespace q35 {
namespace {

// ---------------------------------------------------------------- a small JSON reader
// Enough of JSON for a safetensors header: objects, arrays, strings (with escapes), numbers,
// true / false / null.
struct JVal {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool fail_at(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool parse_str(std::string& out) {
    if (p >= e || *p != '"') return fail_at("expected a string");
    ++p;
    out.clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return fail_at("bad escape");
        switch (*p) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (e - p < 5) return fail_at("bad \\u escape");
            unsigned cp = 0;
            for (int i = 1; i <= 4; ++i) {
              const char c = p[i];
              cp = cp * 16 + (c >= '0' && c <= '9' ? c - '0' : (c | 32) - 'a' + 10);
            }
            p += 4;
            if (cp < 0x80) {
              out += (char)cp;
            } else if (cp < 0x800) {
              out += (char)(0xC0 | (cp >> 6));
              out += (char)(0x80 | (cp & 63));
            } else {
              out += (char)(0xE0 | (cp >> 12));
              out += (char)(0x80 | ((cp >> 6) & 63));
              out += (char)(0x80 | (cp & 63));
            }
          } break;
          default: return fail_at("bad escape");
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail_at("unterminated string");
    ++p;
    return true;
  }
  bool parse(JVal& v, int depth = 0) {
    if (depth > 64) return fail_at("nesting too deep");
    ws();
    if (p >= e) return fail_at("unexpected end");
    if (*p == '{') {
      ++p;
      v.kind = JVal::kObj;
      ws();
      if (p < e && *p == '}') { ++p; return true; }
      while (true) {
        ws();
        std::string k;
        if (!parse_str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail_at("expected ':'");
        ++p;
        JVal c;
        if (!parse(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == '}') { ++p; return true; }
        return fail_at("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      ++p;
      v.kind = JVal::kArr;
      ws();
      if (p < e && *p == ']') { ++p; return true; }
      while (true) {
        JVal c;
        if (!parse(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == ']') { ++p; return true; }
        return fail_at("expected ',' or ']'");
      }
    }
    if (*p == '"') {
      v.kind = JVal::kStr;
      return parse_str(v.str);
    }
    if (e - p >= 4 && !strncmp(p, "true", 4)) { p += 4; v.kind = JVal::kBool; v.num = 1; return true; }
    if (e - p >= 5 && !strncmp(p, "false", 5)) { p += 5; v.kind = JVal::kBool; v.num = 0; return true; }
    if (e - p >= 4 && !strncmp(p, "null", 4)) { p += 4; v.kind = JVal::kNull; return true; }
    const char* s = p;
    while (p < e && (strchr("+-.eE", *p) || (*p >= '0' && *p <= '9'))) ++p;
    if (p == s) return fail_at("unexpected character");
    v.kind = JVal::kNum;
    v.num = strtod(std::string(s, p).c_str(), nullptr);
    return true;
  }
};

float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  const uint32_t sgn = (uint32_t)(h >> 15) << 31;
  const int ex = (h >> 10) & 31;
  uint32_t man = h & 1023;
  uint32_t u;
  if (ex == 0) {
    if (man == 0) {
      u = sgn;
    } else {  // subnormal: renormalise
      int sh = 0;
      while (!(man & 1024)) { man <<= 1; ++sh; }
      man &= 1023;
      u = sgn | ((uint32_t)(127 - 15 - sh + 1) << 23) | (man << 13);
    }
  } else if (ex == 31) {
    u = sgn | 0x7f800000u | (man << 13);
  } else {
    u = sgn | ((uint32_t)(ex - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

struct SafeTensors {
  struct Entry {
    int dtype;  // 0 f32, 1 f16, 2 bf16
    std::vector<int64_t> shape;
    size_t begin, end;
  };
  int fd = -1;
  void* map = MAP_FAILED;
  size_t size = 0;
  const uint8_t* data = nullptr;
  std::map<std::string, Entry> t;

  ~SafeTensors() {
    if (map != MAP_FAILED) munmap(map, size);
    if (fd >= 0) close(fd);
  }

  int open_file(const std::string& path) {
    fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail(Q35_E_ARG, "safetensors: cannot open " + path);
    struct stat stt;
    if (fstat(fd, &stt) != 0 || stt.st_size < 8) return fail(Q35_E_ARG, "safetensors: " + path + " is too short");
    size = (size_t)stt.st_size;
    map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) return fail(Q35_E_NOMEM, "safetensors: mmap failed for " + path);
    const uint8_t* b = static_cast<const uint8_t*>(map);
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i) hl = (hl << 8) | b[i];
    if (hl > size - 8) return fail(Q35_E_ARG, "safetensors: header length past the end of the file");
    JParser jp{reinterpret_cast<const char*>(b + 8), reinterpret_cast<const char*>(b + 8 + hl), {}};
    JVal root;
    if (!jp.parse(root) || root.kind != JVal::kObj) return fail(Q35_E_ARG, "safetensors: bad header JSON (" + jp.err + ")");
    data = b + 8 + hl;
    const size_t avail = size - 8 - hl;
    for (const auto& kv : root.obj) {
      if (kv.first == "__metadata__") continue;
      const JVal* dt = kv.second.get("dtype");
      const JVal* sh = kv.second.get("shape");
      const JVal* off = kv.second.get("data_offsets");
      if (!dt || dt->kind != JVal::kStr || !sh || sh->kind != JVal::kArr || !off || off->kind != JVal::kArr ||
          off->arr.size() != 2)
        return fail(Q35_E_ARG, "safetensors: malformed entry " + kv.first);
      Entry en;
      if (dt->str == "F32") en.dtype = 0;
      else if (dt->str == "F16") en.dtype = 1;
      else if (dt->str == "BF16") en.dtype = 2;
      else en.dtype = -1;  // other dtypes are only an error if the decoder needs the tensor
      int64_t n = 1;
      for (const JVal& s : sh->arr) {
        en.shape.push_back((int64_t)s.num);
        n *= (int64_t)s.num;
      }
      en.begin = (size_t)off->arr[0].num;
      en.end = (size_t)off->arr[1].num;
      const size_t es = en.dtype == 0 ? 4 : 2;
      if (en.end < en.begin || en.end > avail || (en.dtype >= 0 && en.end - en.begin != (size_t)n * es))
        return fail(Q35_E_ARG, "safetensors: data offsets of " + kv.first + " do not match its shape");
      t[kv.first] = en;
    }
    return Q35_OK;
  }

  // The checkpoint key of a decoder tensor: `model.language_model.` + rest, or without the
  // `model.` prefix that the reference strips.
  const Entry* find(const std::string& rest, std::string* key) const {
    for (const char* pre : {"model.language_model.", "language_model."}) {
      auto it = t.find(pre + rest);
      if (it != t.end()) {
        *key = it->first;
        return &it->second;
      }
    }
    return nullptr;
  }

  // n values of `e` as f32, transposed from [a][b] to [b][a] when transpose_ab.
  void read_f32(const Entry& e, float* out, int64_t n, bool transpose, int64_t a, int64_t b) const {
    const uint8_t* src = data + e.begin;
    auto at = [&](int64_t i) -> float {
      if (e.dtype == 0) {
        float f;
        memcpy(&f, src + 4 * i, 4);
        return f;
      }
      uint16_t h;
      memcpy(&h, src + 2 * i, 2);
      return e.dtype == 2 ? bf16_to_f32(h) : f16_to_f32(h);
    };
    if (!transpose) {
      parallel_for(n, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) out[i] = at(i);
      });
    } else {  // 64 x 64 tiles, so both sides are read and written a cache line at a time
      const int64_t tb = (b + 63) / 64;
      parallel_for(((a + 63) / 64) * tb, [&](int64_t lo, int64_t hi) {
        for (int64_t tile = lo; tile < hi; ++tile) {
          const int64_t i0 = (tile / tb) * 64, j0 = (tile % tb) * 64;
          const int64_t i1 = std::min(a, i0 + 64), j1 = std::min(b, j0 + 64);
          for (int64_t i = i0; i < i1; ++i)
            for (int64_t j = j0; j < j1; ++j) out[j * a + i] = at(i * b + j);
        }
      });
    }
  }
};

void SafeTensorsClose::operator()(SafeTensors* s) const { delete s; }

SafeTensorsPtr open_safetensors(const std::string& path, int* rc) {
  SafeTensorsPtr s(new SafeTensors());
  *rc = s->open_file(path);
  if (*rc) s.reset();
  return s;
}

// Values of a decoder tensor in the builder's layout (TensorSpec: rows x cols, Burn's [in][out]
// for Linear weights).  Linear weights (Q8 KN projections, in_proj_b / in_proj_a) are stored by
// PyTorch as [out][in] and transposed; the embedding is [V][H] in both; conv1d.weight is
// [conv_dim][1][k]; vectors are read as they are.
int safetensors_values(const SafeTensors& st, const TensorSpec& t, float* out) {
  const int64_t n = t.rows * t.cols;
  std::string rest = t.name;
  auto ends = [&](const char* sfx) {
    const size_t l = strlen(sfx);
    return rest.size() >= l && rest.compare(rest.size() - l, l, sfx) == 0;
  };
  // the reference's Linear modules: every Q8 projection, and the f32 in_proj_b / in_proj_a
  const bool linear = t.kind == kQ8KN || ends("in_proj_b") || ends("in_proj_a");
  std::string key;
  const SafeTensors::Entry* e = st.find(rest + ".weight", &key);
  if (!e && ends(".a_log"))
    e = st.find(rest.substr(0, rest.size() - 6) + ".A_log", &key);  // `.A_log` -> `.a_log`
  if (!e) e = st.find(rest, &key);
  if (!e) return fail(Q35_E_ARG, "safetensors: tensor " + rest + " not found (looked for model.language_model." + rest + "[.weight])");
  if (e->dtype < 0) return fail(Q35_E_ARG, "safetensors: " + key + " has an unsupported dtype (F32, F16 and BF16 are read)");
  int64_t ne = 1;
  for (int64_t s : e->shape) ne *= s;
  if (ne != n) return fail(Q35_E_SHAPE, "safetensors: " + key + " has " + std::to_string(ne) + " values, the decoder needs " +
                                            std::to_string(n) + " (" + std::to_string(t.rows) + " x " + std::to_string(t.cols) + ")");
  if (linear) {
    if (e->shape.size() != 2 || e->shape[0] != t.cols || e->shape[1] != t.rows)
      return fail(Q35_E_SHAPE, "safetensors: Linear weight " + key + " must be [out=" + std::to_string(t.cols) + "][in=" +
                                   std::to_string(t.rows) + "]");
    st.read_f32(*e, out, n, true, t.cols, t.rows);
  } else {
    if (t.kind == kQ8NK && (e->shape.size() != 2 || e->shape[0] != t.rows || e->shape[1] != t.cols))
      return fail(Q35_E_SHAPE, "safetensors: " + key + " must be [" + std::to_string(t.rows) + "][" + std::to_string(t.cols) + "]");
    st.read_f32(*e, out, n, false, 0, 0);
  }
  if (ends("conv1d")) {
    std::string bkey;
    if (st.find(rest + ".bias", &bkey))
      return fail(Q35_E_ARG, "safetensors: " + bkey + " present; the decoder's causal conv has no bias");
  }
  return Q35_OK;
}

}  // namespace q35

extern "C" int q35_safetensors_tensor(const char* path, const q35_dims* d, const char* name, float* out_host, int64_t n) {
  using namespace q35;
  if (!path || !d || !name || !out_host) return fail(Q35_E_ARG, "safetensors_tensor: null pointer");
  int rc = validate_dims(*d);
  if (rc) return rc;
  for (const TensorSpec& t : model_specs(*d)) {
    if (t.name != name) continue;
    if (n != t.rows * t.cols) return fail(Q35_E_SHAPE, std::string("safetensors_tensor: ") + name + " has " +
                                                            std::to_string(t.rows * t.cols) + " values");
    SafeTensorsPtr st = open_safetensors(path, &rc);
    if (rc) return rc;
    return safetensors_values(*st, t, out_host);
  }
  return fail(Q35_E_ARG, std::string("safetensors_tensor: the decoder has no tensor ") + name);
}
