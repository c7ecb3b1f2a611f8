// On-disk formats (host code): the reference's GRFT graft checkpoint
// (save_safetensors / load_safetensors_checkpoint,
// src/checkpoint_impl.inc:39-97, :170-285), its raw f32 --init-deltas file
// (grafting.hip:882-901) and the base model's safetensors files
// (load_base_model_safetensors, src/model_io_impl.inc:16-190).
//
// GRFT = u32 magic 0x54465247 | u8 version 4 | safetensors body. The
// safetensors body is a u64 little-endian header length, a JSON header and
// the tensor data; its header is parsed here by a small reader of the JSON
// subset safetensors headers use (objects, arrays, strings, integers).
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.hpp"

namespace glt {

namespace {

constexpr uint32_t kGrftMagic = 0x54465247u;  // "GRFT"
constexpr uint8_t kGrftVersion = 4;
constexpr uint64_t kMaxHeader = 100u << 20;

uint16_t rne_bf16(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}
float widen_bf16(uint16_t v) {
  const uint32_t b = (uint32_t)v << 16;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

// ---- JSON subset reader
struct JVal {
  enum Kind { NUL, STR, NUM, OBJ, ARR, BOOL } kind = NUL;
  std::string str;
  int64_t num = 0;
  std::map<std::string, JVal> obj;
  std::vector<JVal> arr;
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
  bool string(std::string& out) {
    if (p >= e || *p != '"') return fail("expected a string");
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return fail("bad escape");
        switch (*p) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {  // code points below 0x80 only (names and metadata here are ASCII)
            if (e - p < 5) return fail("bad \\u escape");
            unsigned v = 0;
            for (int i = 1; i <= 4; ++i) {
              const char c = p[i];
              v = v * 16 + (unsigned)(c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                                      : c >= 'A' && c <= 'F' ? c - 'A' + 10 : 255);
              if (v > 0xFFFF) return fail("bad \\u escape");
            }
            if (v >= 0x80) return fail("non-ASCII \\u escape");
            out += (char)v;
            p += 4;
            break;
          }
          default: return fail("bad escape");
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 16) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    if (*p == '{') {
      v.kind = JVal::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') return ++p, true;
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.obj[k] = std::move(x);
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == '}') return ++p, true;
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      v.kind = JVal::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') return ++p, true;
      for (;;) {
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.arr.push_back(std::move(x));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == ']') return ++p, true;
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') {
      v.kind = JVal::STR;
      return string(v.str);
    }
    if (*p == '-' || (*p >= '0' && *p <= '9')) {
      v.kind = JVal::NUM;
      bool neg = *p == '-';
      if (neg) ++p;
      if (p >= e || *p < '0' || *p > '9') return fail("bad number");
      int64_t x = 0;
      while (p < e && *p >= '0' && *p <= '9') {
        if (x > (INT64_MAX - 9) / 10) return fail("number too large");
        x = x * 10 + (*p++ - '0');
      }
      if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return fail("non-integer number");
      v.num = neg ? -x : x;
      return true;
    }
    auto word = [&](const char* w, JVal::Kind k) {
      const size_t n = std::strlen(w);
      if ((size_t)(e - p) < n || std::strncmp(p, w, n) != 0) return fail("bad literal");
      p += n;
      v.kind = k;
      return true;
    };
    if (*p == 't') return word("true", JVal::BOOL);
    if (*p == 'f') return word("false", JVal::BOOL);
    if (*p == 'n') return word("null", JVal::NUL);
    return fail("unexpected character");
  }
};

bool read_file(const char* path, std::vector<unsigned char>& buf) {
  FILE* f = std::fopen(path, "rb");
  if (!f) return false;
  bool ok = std::fseek(f, 0, SEEK_END) == 0;
  const long n = ok ? std::ftell(f) : -1;
  ok = ok && n >= 0 && std::fseek(f, 0, SEEK_SET) == 0;
  if (ok) {
    buf.resize((size_t)n);
    ok = n == 0 || std::fread(buf.data(), 1, (size_t)n, f) == (size_t)n;
  }
  std::fclose(f);
  return ok;
}

glt_status check_info(const glt_grft_info* d, const char* who) {
  GLT_CHECK(d, GLT_ERR_INVALID_ARG, "%s: null info", who);
  GLT_CHECK(d->num_layers > 0 && d->S > 0 && d->H > 0, GLT_ERR_SHAPE, "%s: num_layers=%d S=%d H=%d", who,
            d->num_layers, d->S, d->H);
  return GLT_OK;
}

int64_t n_elems(const glt_grft_info* d) { return (int64_t)d->num_layers * 3 * d->S * d->H; }

// weight <- host f32 values (device: copied on the stream, then waited for)
glt_status put_weights(float* weight, int on_device, const std::vector<float>& h, hipStream_t st, const char* who) {
  if (!on_device) {
    std::memcpy(weight, h.data(), h.size() * 4);
    return GLT_OK;
  }
  GLT_CHECK(hipMemcpyAsync(weight, h.data(), h.size() * 4, hipMemcpyHostToDevice, st) == hipSuccess &&
                hipStreamSynchronize(st) == hipSuccess,
            GLT_ERR_HIP, "%s: copy to the device failed", who);
  return GLT_OK;
}

// ---- base model files
struct StTensor {
  int dtype;  // GLT_DTYPE_* or -1 (a dtype this loader does not read)
  std::vector<int64_t> shape;
  const unsigned char* data;
  size_t bytes;
};

int st_dtype(const std::string& s) {
  if (s == "BF16") return GLT_DTYPE_BF16;
  if (s == "F32") return GLT_DTYPE_F32;
  if (s == "F16") return GLT_DTYPE_F16;
  return -1;
}
size_t st_esize(int dt) { return dt == GLT_DTYPE_F32 ? 4 : 2; }

// IEEE binary16 -> f32 (exact)
float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t b;
  if (ex == 0x1F) {
    b = sign | 0x7F800000u | (man << 13);
  } else if (ex != 0) {
    b = sign | ((ex + 112) << 23) | (man << 13);
  } else if (man == 0) {
    b = sign;
  } else {  // subnormal: renormalise
    int e = -1;
    uint32_t m = man;
    do {
      ++e;
      m <<= 1;
    } while ((m & 0x400u) == 0);
    b = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3FFu) << 13);
  }
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
uint16_t to_bf16(float f) { return std::isnan(f) ? (uint16_t)0x7FC0u : rne_bf16(f); }

float st_elem(const StTensor& t, size_t i) {
  if (t.dtype == GLT_DTYPE_F32) {
    float f;
    std::memcpy(&f, t.data + 4 * i, 4);
    return f;
  }
  uint16_t h;
  std::memcpy(&h, t.data + 2 * i, 2);
  return t.dtype == GLT_DTYPE_BF16 ? widen_bf16(h) : half_to_f32(h);
}

}  // namespace

}  // namespace glt

// the set of mapped files behind a glt_st_set handle
struct glt_st_set {
  std::vector<std::pair<void*, size_t>> maps;
  std::map<std::string, glt::StTensor> tensors;
};

namespace glt {
namespace {

void st_unmap(glt_st_set* s) {
  for (auto& m : s->maps)
    if (m.first && m.first != MAP_FAILED) munmap(m.first, m.second);
  s->maps.clear();
}

// Maps one file and adds its tensors (names already present stay as they are).
glt_status st_add_file(glt_st_set* s, const std::string& path) {
  const int fd = open(path.c_str(), O_RDONLY);
  GLT_CHECK(fd >= 0, GLT_ERR_IO, "glt_st_open: cannot open %s", path.c_str());
  struct stat stt;
  const bool st_ok = fstat(fd, &stt) == 0;
  const size_t size = st_ok ? (size_t)stt.st_size : 0;
  void* addr = (st_ok && size > 0) ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
  close(fd);
  GLT_CHECK(st_ok && size >= 8, GLT_ERR_FORMAT, "glt_st_open: %s is not a safetensors file", path.c_str());
  GLT_CHECK(addr != MAP_FAILED, GLT_ERR_IO, "glt_st_open: cannot map %s", path.c_str());
  s->maps.emplace_back(addr, size);
  const unsigned char* base = static_cast<const unsigned char*>(addr);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base[i];
  GLT_CHECK(hlen <= kMaxHeader && hlen <= size - 8, GLT_ERR_FORMAT, "glt_st_open: %s: header length %llu",
            path.c_str(), (unsigned long long)hlen);
  JParser jp{reinterpret_cast<const char*>(base + 8), reinterpret_cast<const char*>(base + 8 + hlen), {}};
  JVal root;
  GLT_CHECK(jp.value(root, 0) && root.kind == JVal::OBJ, GLT_ERR_FORMAT, "glt_st_open: %s: header: %s",
            path.c_str(), jp.err.empty() ? "not an object" : jp.err.c_str());
  const size_t data0 = 8 + (size_t)hlen, avail = size - data0;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const JVal& t = kv.second;
    auto dt = t.obj.find("dtype");
    auto sh = t.obj.find("shape");
    auto off = t.obj.find("data_offsets");
    GLT_CHECK(t.kind == JVal::OBJ && dt != t.obj.end() && dt->second.kind == JVal::STR && sh != t.obj.end() &&
                  sh->second.kind == JVal::ARR && off != t.obj.end() && off->second.kind == JVal::ARR &&
                  off->second.arr.size() == 2,
              GLT_ERR_FORMAT, "glt_st_open: %s: tensor %s: malformed entry", path.c_str(), kv.first.c_str());
    StTensor x;
    x.dtype = st_dtype(dt->second.str);
    int64_t n = 1;
    for (const JVal& d : sh->second.arr) {
      GLT_CHECK(d.kind == JVal::NUM && d.num >= 0 && (d.num == 0 || n <= INT64_MAX / d.num), GLT_ERR_FORMAT,
                "glt_st_open: %s: tensor %s: bad shape", path.c_str(), kv.first.c_str());
      x.shape.push_back(d.num);
      n *= d.num;
    }
    const JVal& b = off->second.arr[0];
    const JVal& e = off->second.arr[1];
    GLT_CHECK(b.kind == JVal::NUM && e.kind == JVal::NUM && b.num >= 0 && e.num >= b.num && (size_t)e.num <= avail,
              GLT_ERR_FORMAT, "glt_st_open: %s: tensor %s: data_offsets outside the file", path.c_str(),
              kv.first.c_str());
    x.data = base + data0 + b.num;
    x.bytes = (size_t)(e.num - b.num);
    // n is compared through a division first: the product n * esize could
    // wrap around for a crafted shape and match a small byte count
    if (x.dtype >= 0)
      GLT_CHECK((uint64_t)n <= x.bytes / st_esize(x.dtype) && x.bytes == (size_t)n * st_esize(x.dtype), GLT_ERR_FORMAT,
                "glt_st_open: %s: tensor %s: %zu bytes for %lld elements", path.c_str(), kv.first.c_str(), x.bytes,
                (long long)n);
    s->tensors.emplace(kv.first, std::move(x));
  }
  return GLT_OK;
}

const StTensor* st_find(const glt_st_set* s, const char* name) {
  auto it = s->tensors.find(name);
  return it == s->tensors.end() ? nullptr : &it->second;
}

// the tensor's shape, or GLT_ERR_NOT_FOUND / GLT_ERR_SHAPE against `want`
glt_status st_expect(const glt_st_set* s, const std::string& name, std::vector<int64_t> want, const char* who) {
  const StTensor* t = st_find(s, name.c_str());
  GLT_CHECK(t, GLT_ERR_NOT_FOUND, "%s: %s not found", who, name.c_str());
  GLT_CHECK(t->shape == want, GLT_ERR_SHAPE, "%s: %s has shape of %zu dims, not the expected one", who, name.c_str(),
            t->shape.size());
  return GLT_OK;
}

}  // namespace
}  // namespace glt

using namespace glt;

extern "C" {

glt_status glt_grft_save(const char* path, const glt_grft_info* info, const float* weight, int32_t weight_on_device,
                         void* stream) {
  glt_status s = check_info(info, "glt_grft_save");
  if (s != GLT_OK) return s;
  GLT_CHECK(path && weight, GLT_ERR_INVALID_ARG, "glt_grft_save: null path/weight");
  const int64_t n = n_elems(info);
  std::vector<float> h((size_t)n);
  if (weight_on_device) {
    hipStream_t st = as_stream(stream);
    GLT_CHECK(hipMemcpyAsync(h.data(), weight, (size_t)n * 4, hipMemcpyDeviceToHost, st) == hipSuccess &&
                  hipStreamSynchronize(st) == hipSuccess,
              GLT_ERR_HIP, "glt_grft_save: copy from the device failed");
  } else {
    std::memcpy(h.data(), weight, (size_t)n * 4);
  }
  std::vector<uint16_t> b((size_t)n);
  for (int64_t i = 0; i < n; ++i) b[(size_t)i] = rne_bf16(h[(size_t)i]);

  // header in the reference's key order and spelling (src/checkpoint_impl.inc:16-35)
  const std::string sid = info->session_id ? info->session_id : "";
  for (char c : sid)
    GLT_CHECK(c != '"' && c != '\\' && (unsigned char)c >= 0x20, GLT_ERR_INVALID_ARG,
              "glt_grft_save: session_id needs JSON escaping (not written by the reference format)");
  const int64_t bytes = n * 2;
  auto q = [](long long v) { return "\"" + std::to_string(v) + "\""; };
  std::string header = "{\"__metadata__\":{\"session_id\":\"" + sid + "\",\"domain_id\":" + q(info->domain_id) +
                       ",\"slice_dim\":" + q(info->S) + ",\"h_slice_dim\":" + q(info->H) +
                       ",\"hidden_dim\":" + q(info->hidden_dim) + ",\"num_layers\":" + q(info->num_layers) +
                       "},\"delta_weights\":{\"dtype\":\"BF16\",\"shape\":[" +
                       std::to_string((long long)info->num_layers * 3) + "," + std::to_string(info->S) + "," +
                       std::to_string(info->H) + "],\"data_offsets\":[0," + std::to_string((long long)bytes) + "]}}";
  const uint64_t padded = (header.size() + 7) / 8 * 8;

  FILE* f = std::fopen(path, "wb");
  GLT_CHECK(f, GLT_ERR_IO, "glt_grft_save: cannot open %s for writing", path);
  const uint32_t magic = kGrftMagic;
  const uint8_t ver = kGrftVersion;
  const std::vector<char> pad(padded - header.size(), '\0');
  bool ok = std::fwrite(&magic, 4, 1, f) == 1 && std::fwrite(&ver, 1, 1, f) == 1 &&
            std::fwrite(&padded, 8, 1, f) == 1 && std::fwrite(header.data(), 1, header.size(), f) == header.size() &&
            (pad.empty() || std::fwrite(pad.data(), 1, pad.size(), f) == pad.size()) &&
            std::fwrite(b.data(), 2, b.size(), f) == b.size();
  ok = (std::fclose(f) == 0) && ok;
  GLT_CHECK(ok, GLT_ERR_IO, "glt_grft_save: short write to %s", path);
  return GLT_OK;
}

glt_status glt_grft_load(const char* path, const glt_grft_info* expect, float* weight, int32_t weight_on_device,
                         void* stream) {
  glt_status s = check_info(expect, "glt_grft_load");
  if (s != GLT_OK) return s;
  GLT_CHECK(path && weight, GLT_ERR_INVALID_ARG, "glt_grft_load: null path/weight");
  std::vector<unsigned char> buf;
  GLT_CHECK(read_file(path, buf), GLT_ERR_IO, "glt_grft_load: cannot read %s", path);
  size_t base = 0;
  uint32_t magic = 0;
  if (buf.size() >= 5) std::memcpy(&magic, buf.data(), 4);
  if (magic == kGrftMagic) base = 5;  // version byte not checked, as the reference (:187-193)
  GLT_CHECK(buf.size() >= base + 8, GLT_ERR_FORMAT, "glt_grft_load: %s is too short for a header", path);
  uint64_t hlen = 0;
  std::memcpy(&hlen, buf.data() + base, 8);
  GLT_CHECK(hlen <= kMaxHeader && base + 8 + hlen <= buf.size(), GLT_ERR_FORMAT,
            "glt_grft_load: header length %llu does not fit %s", (unsigned long long)hlen, path);
  const char* hb = reinterpret_cast<const char*>(buf.data() + base + 8);
  size_t hn = (size_t)hlen;
  while (hn > 0 && (hb[hn - 1] == '\0' || hb[hn - 1] == ' ')) --hn;  // NUL (reference) or space padding
  JParser jp{hb, hb + hn, {}};
  JVal root;
  bool ok = jp.value(root, 0);
  jp.ws();
  GLT_CHECK(ok && jp.p == jp.e && root.kind == JVal::OBJ, GLT_ERR_FORMAT, "glt_grft_load: bad header in %s: %s",
            path, jp.err.empty() ? "trailing data" : jp.err.c_str());
  auto it = root.obj.find("delta_weights");
  GLT_CHECK(it != root.obj.end() && it->second.kind == JVal::OBJ, GLT_ERR_FORMAT,
            "glt_grft_load: 'delta_weights' not found in %s", path);
  const JVal& t = it->second;
  auto dt = t.obj.find("dtype"), sh = t.obj.find("shape"), off = t.obj.find("data_offsets");
  GLT_CHECK(dt != t.obj.end() && dt->second.kind == JVal::STR && dt->second.str == "BF16", GLT_ERR_FORMAT,
            "glt_grft_load: delta_weights dtype is not BF16");
  const int64_t want[3] = {(int64_t)expect->num_layers * 3, expect->S, expect->H};
  ok = sh != t.obj.end() && sh->second.kind == JVal::ARR && sh->second.arr.size() == 3;
  for (int i = 0; ok && i < 3; ++i) ok = sh->second.arr[i].kind == JVal::NUM && sh->second.arr[i].num == want[i];
  GLT_CHECK(ok, GLT_ERR_FORMAT, "glt_grft_load: delta_weights shape is not [%lld,%lld,%lld]", (long long)want[0],
            (long long)want[1], (long long)want[2]);
  const int64_t n = n_elems(expect);
  const uint64_t data0 = base + 8 + hlen;
  ok = off != t.obj.end() && off->second.kind == JVal::ARR && off->second.arr.size() == 2 &&
       off->second.arr[0].kind == JVal::NUM && off->second.arr[1].kind == JVal::NUM;
  const int64_t b0 = ok ? off->second.arr[0].num : 0, b1 = ok ? off->second.arr[1].num : 0;
  GLT_CHECK(ok && b0 >= 0 && b1 - b0 == n * 2 && data0 + (uint64_t)b1 <= buf.size(), GLT_ERR_FORMAT,
            "glt_grft_load: delta_weights data_offsets do not match %lld bf16 values in the file", (long long)n);

  // metadata checks (reference :219-246)
  std::string file_sid;
  int64_t file_domain = -1;
  auto md = root.obj.find("__metadata__");
  if (md != root.obj.end() && md->second.kind == JVal::OBJ) {
    auto a = md->second.obj.find("session_id");
    if (a != md->second.obj.end() && a->second.kind == JVal::STR) file_sid = a->second.str;
    auto b = md->second.obj.find("domain_id");
    if (b != md->second.obj.end() && b->second.kind == JVal::STR) {
      char* endp = nullptr;
      const long long v = std::strtoll(b->second.str.c_str(), &endp, 10);
      GLT_CHECK(endp && *endp == '\0' && !b->second.str.empty(), GLT_ERR_FORMAT,
                "glt_grft_load: domain_id '%s' is not an integer", b->second.str.c_str());
      file_domain = v;
    }
  }
  const std::string want_sid = expect->session_id ? expect->session_id : "";
  GLT_CHECK(want_sid.empty() || file_sid.empty() || want_sid == file_sid, GLT_ERR_FORMAT,
            "glt_grft_load: session_id mismatch (file '%s', expected '%s'): grafts from different training runs "
            "cannot be mixed", file_sid.c_str(), want_sid.c_str());
  GLT_CHECK(file_domain == -1 || file_domain == expect->domain_id, GLT_ERR_FORMAT,
            "glt_grft_load: domain_id mismatch (file %lld, expected %d)", (long long)file_domain,
            expect->domain_id);

  std::vector<float> h((size_t)n);
  const unsigned char* src = buf.data() + data0 + b0;
  for (int64_t i = 0; i < n; ++i) {
    uint16_t v;
    std::memcpy(&v, src + 2 * i, 2);
    h[(size_t)i] = widen_bf16(v);
  }
  return put_weights(weight, weight_on_device, h, as_stream(stream), "glt_grft_load");
}

glt_status glt_grft_load_raw_f32(const char* path, const glt_grft_info* expect, float* weight,
                                 int32_t weight_on_device, void* stream) {
  glt_status s = check_info(expect, "glt_grft_load_raw_f32");
  if (s != GLT_OK) return s;
  GLT_CHECK(path && weight, GLT_ERR_INVALID_ARG, "glt_grft_load_raw_f32: null path/weight");
  std::vector<unsigned char> buf;
  GLT_CHECK(read_file(path, buf), GLT_ERR_IO, "glt_grft_load_raw_f32: cannot read %s", path);
  const int64_t n = n_elems(expect);
  GLT_CHECK((int64_t)buf.size() == n * 4, GLT_ERR_FORMAT, "glt_grft_load_raw_f32: %s has %zu bytes, expected %lld",
            path, buf.size(), (long long)n * 4);
  std::vector<float> h((size_t)n);
  std::memcpy(h.data(), buf.data(), buf.size());
  return put_weights(weight, weight_on_device, h, as_stream(stream), "glt_grft_load_raw_f32");
}

glt_status glt_st_open(const char* path, glt_st_set** out) {
  GLT_CHECK(path && out, GLT_ERR_INVALID_ARG, "glt_st_open: null path/out");
  *out = nullptr;
  struct stat st;
  GLT_CHECK(stat(path, &st) == 0, GLT_ERR_IO, "glt_st_open: %s does not exist", path);
  std::vector<std::string> files;
  if (S_ISREG(st.st_mode)) {
    files.push_back(path);
  } else if (S_ISDIR(st.st_mode)) {
    DIR* d = opendir(path);
    GLT_CHECK(d, GLT_ERR_IO, "glt_st_open: cannot list %s", path);
    const std::string ext = ".safetensors";
    for (dirent* e = readdir(d); e; e = readdir(d)) {
      const std::string n = e->d_name;
      if (n.size() <= ext.size() || n.compare(n.size() - ext.size(), ext.size(), ext) != 0) continue;
      const std::string full = std::string(path) + "/" + n;
      struct stat fs;
      if (stat(full.c_str(), &fs) == 0 && S_ISREG(fs.st_mode)) files.push_back(full);
    }
    closedir(d);
    std::sort(files.begin(), files.end());
  }
  GLT_CHECK(!files.empty(), GLT_ERR_IO, "glt_st_open: no .safetensors files at %s", path);
  glt_st_set* s = new glt_st_set();
  for (const std::string& f : files) {
    const glt_status r = st_add_file(s, f);
    if (r != GLT_OK) {
      st_unmap(s);
      delete s;
      return r;
    }
  }
  *out = s;
  return GLT_OK;
}

void glt_st_close(glt_st_set* s) {
  if (!s) return;
  st_unmap(s);
  delete s;
}

int32_t glt_st_count(const glt_st_set* s) { return s ? (int32_t)s->tensors.size() : 0; }

glt_status glt_st_info(const glt_st_set* s, const char* name, int32_t* dtype, int32_t* ndim, int64_t* shape) {
  GLT_CHECK(s && name, GLT_ERR_INVALID_ARG, "glt_st_info: null set/name");
  const StTensor* t = st_find(s, name);
  GLT_CHECK(t, GLT_ERR_NOT_FOUND, "glt_st_info: %s not found", name);
  GLT_CHECK(t->dtype >= 0, GLT_ERR_DTYPE, "glt_st_info: %s has a dtype this loader does not read", name);
  GLT_CHECK(t->shape.size() <= 8, GLT_ERR_SHAPE, "glt_st_info: %s has %zu dims", name, t->shape.size());
  if (dtype) *dtype = t->dtype;
  if (ndim) *ndim = (int32_t)t->shape.size();
  if (shape)
    for (size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
  return GLT_OK;
}

glt_status glt_st_read(const glt_st_set* s, const char* name, void* dst, int32_t dst_dtype, int32_t transpose,
                       int32_t on_device, void* stream) {
  GLT_CHECK(s && name && dst, GLT_ERR_INVALID_ARG, "glt_st_read: null set/name/dst");
  const StTensor* t = st_find(s, name);
  GLT_CHECK(t, GLT_ERR_NOT_FOUND, "glt_st_read: %s not found", name);
  GLT_CHECK(t->dtype >= 0, GLT_ERR_DTYPE, "glt_st_read: %s has a dtype this loader does not read", name);
  GLT_CHECK(dst_dtype == GLT_DTYPE_BF16 || dst_dtype == GLT_DTYPE_F32, GLT_ERR_DTYPE,
            "glt_st_read: destination dtype %d", dst_dtype);
  GLT_CHECK(!transpose || t->shape.size() == 2, GLT_ERR_SHAPE, "glt_st_read: transpose of a %zu-dim tensor",
            t->shape.size());
  // element count and output size with overflow checks (glt_st_open has
  // already tied the count to the stored bytes; this keeps glt_st_read safe
  // on its own)
  size_t n = 1;
  for (int64_t d : t->shape) {
    GLT_CHECK(d >= 0 && (d == 0 || n <= SIZE_MAX / (size_t)d), GLT_ERR_FORMAT, "glt_st_read: %s: shape overflows",
              name);
    n *= (size_t)d;
  }
  GLT_CHECK(n <= t->bytes / st_esize(t->dtype) && n <= SIZE_MAX / 4, GLT_ERR_FORMAT,
            "glt_st_read: %s: %zu elements in %zu stored bytes", name, n, t->bytes);
  const size_t out_bytes = n * st_esize(dst_dtype);
  const unsigned char* src = t->data;
  std::vector<unsigned char> stage;
  if (t->dtype != dst_dtype || (transpose && n > 0)) {
    stage.resize(out_bytes);
    const size_t rows = transpose ? (size_t)t->shape[0] : 1, cols = transpose ? (size_t)t->shape[1] : n;
    for (size_t r = 0; r < rows; ++r)
      for (size_t c = 0; c < cols; ++c) {
        const size_t i = r * cols + c, o = transpose ? c * rows + r : i;
        if (t->dtype == dst_dtype) {
          std::memcpy(stage.data() + o * st_esize(dst_dtype), t->data + i * st_esize(dst_dtype), st_esize(dst_dtype));
        } else if (dst_dtype == GLT_DTYPE_BF16) {
          const uint16_t v = to_bf16(st_elem(*t, i));
          std::memcpy(stage.data() + 2 * o, &v, 2);
        } else {
          const float v = st_elem(*t, i);
          std::memcpy(stage.data() + 4 * o, &v, 4);
        }
      }
    src = stage.data();
  }
  if (out_bytes == 0) return GLT_OK;
  if (!on_device) {
    std::memcpy(dst, src, out_bytes);
    return GLT_OK;
  }
  hipStream_t st = as_stream(stream);
  GLT_CHECK(hipMemcpyAsync(dst, src, out_bytes, hipMemcpyHostToDevice, st) == hipSuccess &&
                hipStreamSynchronize(st) == hipSuccess,
            GLT_ERR_HIP, "glt_st_read: copy of %s to the device failed", name);
  return GLT_OK;
}

glt_status glt_st_load_layer(const glt_st_set* s, int32_t layer, const glt_layer_desc* d,
                             const glt_layer_buffers* dst, int32_t on_device, void* stream) {
  GLT_CHECK(s && d && dst && layer >= 0, GLT_ERR_INVALID_ARG, "glt_st_load_layer: null argument or layer < 0");
  const int64_t D = d->mlp.D, I = d->mlp.I, nq = (int64_t)d->n_q_heads * d->head_dim,
                nk = (int64_t)d->n_kv_heads * d->head_dim;
  const std::string p = "model.layers." + std::to_string(layer) + ".";
  struct Item {
    const char* suffix;
    std::vector<int64_t> shape;
    void* out;
  };
  const Item items[9] = {{"input_layernorm.weight", {D}, dst->ln_in},
                         {"self_attn.q_proj.weight", {nq, D}, dst->q_proj},
                         {"self_attn.k_proj.weight", {nk, D}, dst->k_proj},
                         {"self_attn.v_proj.weight", {nk, D}, dst->v_proj},
                         {"self_attn.o_proj.weight", {D, nq}, dst->o_proj},
                         {"post_attention_layernorm.weight", {D}, dst->ln_post},
                         {"mlp.gate_proj.weight", {I, D}, dst->gate},
                         {"mlp.up_proj.weight", {I, D}, dst->up},
                         {"mlp.down_proj.weight", {D, I}, dst->down}};
  // every tensor is checked before any is copied
  for (const Item& it : items) {
    const glt_status r = st_expect(s, p + it.suffix, it.shape, "glt_st_load_layer");
    if (r != GLT_OK) return r;
  }
  for (const Item& it : items) {
    if (!it.out) continue;
    const glt_status r = glt_st_read(s, (p + it.suffix).c_str(), it.out, GLT_DTYPE_BF16, 0, on_device, stream);
    if (r != GLT_OK) return r;
  }
  return GLT_OK;
}

glt_status glt_st_load_head(const glt_st_set* s, int32_t V, int32_t D, void* embed, void* final_norm, void* lm_head,
                            int32_t on_device, void* stream) {
  GLT_CHECK(s && V > 0 && D > 0, GLT_ERR_INVALID_ARG, "glt_st_load_head: null set or V/D <= 0");
  const char* kEmbed = "model.embed_tokens.weight";
  const char* kNorm = "model.norm.weight";
  const char* kHead = "lm_head.weight";
  glt_status r = st_expect(s, kEmbed, {V, D}, "glt_st_load_head");
  if (r != GLT_OK) return r;
  if ((r = st_expect(s, kNorm, {D}, "glt_st_load_head")) != GLT_OK) return r;
  // lm_head: [V,D] as is (also the square case), [D,V] transposed, absent = tied
  const StTensor* h = st_find(s, kHead);
  const char* head_src = kEmbed;
  int transpose = 0;
  if (h) {
    const std::vector<int64_t> vd{V, D}, dv{D, V};
    GLT_CHECK(h->shape == vd || h->shape == dv, GLT_ERR_SHAPE, "glt_st_load_head: lm_head.weight is neither [%d,%d] "
              "nor [%d,%d]", V, D, D, V);
    head_src = kHead;
    transpose = h->shape == vd ? 0 : 1;
  }
  if (embed && (r = glt_st_read(s, kEmbed, embed, GLT_DTYPE_BF16, 0, on_device, stream)) != GLT_OK) return r;
  if (final_norm && (r = glt_st_read(s, kNorm, final_norm, GLT_DTYPE_BF16, 0, on_device, stream)) != GLT_OK) return r;
  if (lm_head && (r = glt_st_read(s, head_src, lm_head, GLT_DTYPE_BF16, transpose, on_device, stream)) != GLT_OK)
    return r;
  return GLT_OK;
}

}  // extern "C"
