// decide-weights-v1 loader: fills a dh_model's tensors from a converted
// weights directory (decide: Weights::open, crates/decide-engine/src/
// weights.rs:105-183; format written by convert.rs:140-200, 300-400).
//
// The directory holds `decide-index.json` ({"format": "decide-weights-v1",
// "blobs": [...], "tensors": {name: {"blob", "offset", "dtype", "shape"}}})
// and the blobs it names: little-endian tensor bytes at 16 KiB-aligned
// offsets. decide maps the blobs and hands them to Metal without a copy;
// here every blob is mapped read-only and each tensor the model needs is
// copied once into its device buffer (HBM is the working set on MI355X).
// The checks are decide's: the format tag, known dtypes, aligned offsets,
// tensors inside their blob; plus that each tensor matches the model's own
// dtype and element count.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/decide_hip.h"
#include "api_internal.h"

using namespace dh_api;

namespace {

constexpr uint64_t kAlign = 16 * 1024;  // convert.rs:21

// ---- a small JSON reader for the index (objects, arrays, strings, numbers, literals)
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  bool b = false;
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;
  const Json* get(const std::string& k) const {
    if (kind != Obj) return nullptr;
    auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
};

struct Parser {
  const char* p;
  const char* end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(end - p) < n || strncmp(p, s, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool string(std::string& out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) return fail("bad escape");
        const char c = *p++;
        switch (c) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u':  // the index holds ASCII names; keep other code points as '?'
            if (end - p < 4) return fail("bad \\u escape");
            p += 4;
            out += '?';
            break;
          default: out += c;
        }
      } else {
        out += *p++;
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    const char c = *p;
    if (c == '{') {
      v.kind = Json::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') return ++p, true;
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        if (!value(v.obj[k], depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') return ++p, true;
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Json::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') return ++p, true;
      for (;;) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') return ++p, true;
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      return string(v.str);
    }
    if (c == 't') return v.kind = Json::Bool, v.b = true, lit("true");
    if (c == 'f') return v.kind = Json::Bool, v.b = false, lit("false");
    if (c == 'n') return v.kind = Json::Null, lit("null");
    char* q = nullptr;
    const std::string num(p, (size_t)std::min<ptrdiff_t>(end - p, 64));
    v.num = strtod(num.c_str(), &q);
    if (q == num.c_str()) return fail("bad value");
    v.kind = Json::Num;
    p += (q - num.c_str());
    return true;
  }
};

struct Mapped {
  void* ptr = MAP_FAILED;
  size_t len = 0;
  ~Mapped() {
    if (ptr != MAP_FAILED && len) munmap(ptr, len);
  }
};

bool read_file(const std::string& path, std::string& out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
  fclose(f);
  return true;
}

uint32_t dtype_code(const std::string& s, bool& ok) {
  ok = true;
  if (s == "f16") return 0;
  if (s == "bf16") return 1;
  if (s == "f32") return 2;
  ok = false;
  return 0;
}

}  // namespace

extern "C" {

int dh_model_load(dh_model* model, const char* dir) {
  if (!model || !dir) return fail(DH_EINVAL, "model_load: null model or directory");
  const std::string root(dir);
  std::string text;
  const std::string index_path = root + "/decide-index.json";
  if (!read_file(index_path, text)) return fail(DH_EINVAL, "%s does not exist; run `decide convert`", index_path.c_str());
  Json index;
  Parser ps{text.data(), text.data() + text.size(), {}};
  if (!ps.value(index, 0)) return fail(DH_EINVAL, "%s: %s", index_path.c_str(), ps.err.c_str());
  const Json* fmt = index.get("format");
  if (!fmt || fmt->kind != Json::Str || fmt->str != "decide-weights-v1")
    return fail(DH_EINVAL, "%s has format %s; expected decide-weights-v1", index_path.c_str(),
                fmt && fmt->kind == Json::Str ? fmt->str.c_str() : "(none)");
  const Json* blobs = index.get("blobs");
  const Json* tensors = index.get("tensors");
  if (!blobs || blobs->kind != Json::Arr) return fail(DH_EINVAL, "the index has no blob list");
  if (!tensors || tensors->kind != Json::Obj) return fail(DH_EINVAL, "the index has no tensor table");

  std::map<std::string, std::unique_ptr<Mapped>> maps;
  for (const Json& b : blobs->arr) {
    if (b.kind != Json::Str) return fail(DH_EINVAL, "a blob name is not a string");
    const std::string path = root + "/" + b.str;
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail(DH_EINVAL, "opening %s failed", path.c_str());
    struct stat st;
    auto m = std::make_unique<Mapped>();
    if (fstat(fd, &st) == 0 && st.st_size > 0) {
      m->len = (size_t)st.st_size;
      m->ptr = mmap(nullptr, m->len, PROT_READ, MAP_PRIVATE, fd, 0);
    }
    close(fd);
    if (m->ptr == MAP_FAILED && m->len) return fail(DH_EINVAL, "mapping %s failed", path.c_str());
    maps[b.str] = std::move(m);
  }

  // every tensor the model holds must be in the index, with its dtype and size
  for (uint32_t i = 0;; ++i) {
    const char* name = dh_model_tensor_name(model, i);
    if (!name) break;
    void* dst = nullptr;
    uint64_t elems = 0;
    uint32_t dtype = 0;
    if (dh_model_tensor(model, name, &dst, &elems, &dtype) != DH_OK) return DH_EINVAL;
    const Json* e = tensors->get(name);
    if (!e || e->kind != Json::Obj) return fail(DH_EINVAL, "the index has no tensor %s", name);
    const Json* jb = e->get("blob");
    const Json* jo = e->get("offset");
    const Json* jd = e->get("dtype");
    const Json* js = e->get("shape");
    if (!jb || jb->kind != Json::Str) return fail(DH_EINVAL, "tensor %s: missing or bad blob", name);
    // Offsets and dims are JSON numbers (doubles): only integral values up to 2^53 convert to u64 exactly
    // (decide reads them with as_u64, weights.rs:160-171).
    auto exact_u64 = [](const Json* j) {
      return j && j->kind == Json::Num && j->num >= 0 && j->num <= 9007199254740992.0 && std::floor(j->num) == j->num;
    };
    if (!exact_u64(jo)) return fail(DH_EINVAL, "tensor %s: missing or bad offset", name);
    if (!jd || jd->kind != Json::Str) return fail(DH_EINVAL, "tensor %s: missing or bad dtype", name);
    if (!js || js->kind != Json::Arr) return fail(DH_EINVAL, "tensor %s: missing or bad shape", name);
    bool known = false;
    const uint32_t code = dtype_code(jd->str, known);
    if (!known) return fail(DH_EINVAL, "tensor %s: unknown dtype \"%s\"", name, jd->str.c_str());
    if (code != dtype) return fail(DH_EINVAL, "tensor %s is %s; the model holds it as dtype %u", name, jd->str.c_str(), dtype);
    uint64_t n = 1;
    for (const Json& d : js->arr) {
      if (!exact_u64(&d)) return fail(DH_EINVAL, "tensor %s: missing or bad shape", name);
      if (__builtin_mul_overflow(n, (uint64_t)d.num, &n))
        return fail(DH_EINVAL, "tensor %s: shape element count overflows", name);
    }
    if (n != elems) return fail(DH_EINVAL, "tensor %s has %llu elements; the model expects %llu", name,
                                (unsigned long long)n, (unsigned long long)elems);
    const uint64_t off = (uint64_t)jo->num;
    if (off % kAlign != 0) return fail(DH_EINVAL, "tensor %s: offset %llu is not %llu-byte aligned", name,
                                       (unsigned long long)off, (unsigned long long)kAlign);
    auto it = maps.find(jb->str);
    if (it == maps.end())
      return fail(DH_EINVAL, "tensor %s is in %s, which is not in the blob list", name, jb->str.c_str());
    const uint64_t bytes = elems * (dtype == 2 ? 4 : 2);
    if (off > it->second->len || bytes > it->second->len - off) return fail(DH_EINVAL, "tensor %s runs past the end of %s", name, jb->str.c_str());
    const hipError_t err = hipMemcpy(dst, (const char*)it->second->ptr + off, bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) return fail(DH_EDEVICE, "model_load: copying %s: %s", name, hipGetErrorString(err));
  }
  return ok();
}

}  // extern "C"
