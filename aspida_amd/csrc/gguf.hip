// gguf.hip -- GGUF tensor-layout reader (host code only): the header,
// metadata and tensor descriptors of a model file, with the reference's
// validation rules, so that real K-quant weights can be located, checked and
// handed to the packed kernels.
//
// Follows LLM_GGUF.Open_From_Source (src/llm/llm_gguf.adb:317-560): magic
// "GGUF"; version 2 or 3 (others are reported and still parsed); tensor and
// metadata counts capped at 16384, strings at 1 MiB, arrays at 1048576
// elements (28-31); at most 4 dims per tensor; "general.alignment" accepted
// only as a power of two in 1 .. 65536, else 32 (433-455); tensor data from
// the header end rounded up to the alignment (500-506); every tensor's
// [data start + offset, + byte size) inside the file, with overflow-checked
// arithmetic (529-546).  Byte sizes follow Checked_Byte_Size (238-258),
// including its rule that unlisted types count 4 bytes per element; type
// codes follow To_GGML_Type (266-291) and the kind codes LLM_Weight.Kind_Code
// (src/llm/llm_weight.adb:277-292).
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/aspidagpu.h"

namespace {

constexpr uint64_t MAX_STRING = 1048576, MAX_META = 16384, MAX_TENSORS = 16384, MAX_ARRAY = 1048576;
constexpr int MAX_NEST = 8;  // bounds the recursion a hostile file could ask for

struct Tensor {
  std::string name;
  int ggml_type = 0, n_dims = 0;
  uint64_t dims[4] = {0, 0, 0, 0};
  uint64_t offset = 0, bytes = 0;
};

struct Meta {
  std::string key, value;
  int type = 0;
};

struct Reader {
  FILE* f = nullptr;
  uint64_t pos = 0;
  bool ok = true;
  std::string err;
  void fail(const std::string& e) {
    if (ok) err = e;
    ok = false;
  }
  bool read(void* dst, size_t n) {
    if (!ok) return false;
    if (n && fread(dst, 1, n, f) != n) {
      fail("short read at byte " + std::to_string(pos));
      return false;
    }
    pos += n;
    return true;
  }
  template <class T> T get() {
    T v{};
    read(&v, sizeof(T));
    return v;  // little-endian on this host, as GGUF is
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok) return {};
    if (n > MAX_STRING) {
      fail("string of " + std::to_string(n) + " bytes exceeds the 1 MiB cap");
      return {};
    }
    std::string s(n, '\0');
    read(&s[0], n);
    return s;
  }
};

bool checked_mul(uint64_t a, uint64_t b, uint64_t& out) {
  if (a && b > UINT64_MAX / a) return false;
  out = a * b;
  return true;
}

// Checked_Byte_Size (llm_gguf.adb:238-258).
bool byte_size(int type, uint64_t n, uint64_t& out) {
  switch (type) {
    case 0: return checked_mul(n, 4, out);                       // F32
    case 1: return checked_mul(n, 2, out);                       // F16
    case 30: return checked_mul(n, 2, out);                      // BF16
    case 2: return checked_mul((n + 31) / 32, 18, out);          // Q4_0
    case 6: return checked_mul((n + 31) / 32, 22, out);          // Q5_0
    case 7: return checked_mul((n + 31) / 32, 24, out);          // Q5_1
    case 10: return checked_mul((n + 255) / 256, 84, out);       // Q2_K
    case 11: return checked_mul((n + 255) / 256, 110, out);      // Q3_K
    case 12: return checked_mul((n + 255) / 256, 144, out);      // Q4_K
    case 13: return checked_mul((n + 255) / 256, 176, out);      // Q5_K
    case 14: return checked_mul((n + 255) / 256, 210, out);      // Q6_K
    case 15: return checked_mul((n + 255) / 256, 292, out);      // Q8_K
    case 8: return checked_mul((n + 31) / 32, 34, out);          // Q8_0
    default: return checked_mul(n, 4, out);                      // as the reference: 4 bytes per element
  }
}

// GGML type code -> this library's kind code (0 Q4_K, 1 Q6_K, 2 Q5_K, 3 Q3_K,
// 4 Q2_K, 5 Q8_0), -1 for every other type.
int kind_of(int ggml_type) {
  switch (ggml_type) {
    case 12: return 0;
    case 14: return 1;
    case 13: return 2;
    case 11: return 3;
    case 10: return 4;
    case 8: return 5;
    default: return -1;
  }
}

// A metadata value as text.  Arrays read element by element (nested ones too,
// as Read_Metadata_Value recurses, llm_gguf.adb:173-186) and render as
// "[e1, e2, ...]"; the tokenizer's token and merge lists, which the reference
// keeps apart (llm_gguf.adb:384-412), render as "[array: N]".
std::string read_value(Reader& r, uint32_t type, bool summarize = false, int depth = 0) {
  char buf[64];
  switch (type) {
    case 0: snprintf(buf, sizeof buf, "%u", (unsigned)r.get<uint8_t>()); return buf;
    case 1: snprintf(buf, sizeof buf, "%d", (int)r.get<int8_t>()); return buf;
    case 2: snprintf(buf, sizeof buf, "%u", (unsigned)r.get<uint16_t>()); return buf;
    case 3: snprintf(buf, sizeof buf, "%d", (int)r.get<int16_t>()); return buf;
    case 4: snprintf(buf, sizeof buf, "%u", r.get<uint32_t>()); return buf;
    case 5: snprintf(buf, sizeof buf, "%d", r.get<int32_t>()); return buf;
    case 6: snprintf(buf, sizeof buf, "%.9g", (double)r.get<float>()); return buf;
    case 7: return r.get<uint8_t>() ? "true" : "false";
    case 8: return r.str();
    case 10: snprintf(buf, sizeof buf, "%llu", (unsigned long long)r.get<uint64_t>()); return buf;
    case 11: snprintf(buf, sizeof buf, "%lld", (long long)r.get<int64_t>()); return buf;
    case 12: snprintf(buf, sizeof buf, "%.17g", r.get<double>()); return buf;
    case 9: {
      const uint32_t et = r.get<uint32_t>();
      const uint64_t n = r.get<uint64_t>();
      if (!r.ok) return {};
      if (n > MAX_ARRAY) {
        r.fail("metadata array of " + std::to_string(n) + " elements exceeds the cap");
        return {};
      }
      if (depth >= MAX_NEST) {
        r.fail("metadata arrays nested deeper than " + std::to_string(MAX_NEST));
        return {};
      }
      std::string out = summarize ? "" : "[";
      for (uint64_t i = 0; i < n && r.ok; ++i) {
        std::string e = read_value(r, et, summarize, depth + 1);
        if (!summarize) out += (i ? ", " : "") + e;
      }
      return summarize ? "[array: " + std::to_string(n) + "]" : out + "]";
    }
    default:
      r.fail("unknown metadata value type " + std::to_string(type));
      return {};
  }
}

}  // namespace

struct aspida_gguf {
  std::string path;
  uint32_t version = 0;
  uint64_t alignment = 32, data_start = 0, file_size = 0;
  std::vector<Meta> meta;
  std::vector<Tensor> tensors;
};

static std::string g_gguf_err;

extern "C" aspida_gguf* aspida_gguf_open(const char* path) {
  g_gguf_err.clear();
  if (!path) {
    g_gguf_err = "null path";
    return nullptr;
  }
  Reader r;
  r.f = fopen(path, "rb");
  if (!r.f) {
    g_gguf_err = std::string("cannot open ") + path + ": " + strerror(errno);
    return nullptr;
  }
  auto* g = new aspida_gguf();
  g->path = path;
  char magic[4] = {0, 0, 0, 0};
  r.read(magic, 4);
  if (r.ok && memcmp(magic, "GGUF", 4) != 0) r.fail("not a GGUF file (bad magic)");
  g->version = r.get<uint32_t>();
  if (r.ok && g->version != 2 && g->version != 3)
    fprintf(stderr, "[aspida_gguf] GGUF version %u (expected v2 or v3)\n", g->version);
  const uint64_t n_tensors = r.get<uint64_t>(), n_meta = r.get<uint64_t>();
  if (r.ok && (n_tensors > MAX_TENSORS || n_meta > MAX_META))
    r.fail("header reports " + std::to_string(n_tensors) + " tensors / " + std::to_string(n_meta) +
           " metadata (exceeds the 16384 cap)");
  for (uint64_t i = 0; i < n_meta && r.ok; ++i) {
    Meta m;
    m.key = r.str();
    m.type = (int)r.get<uint32_t>();
    m.value = read_value(r, (uint32_t)m.type, m.key == "tokenizer.ggml.tokens" || m.key == "tokenizer.ggml.merges");
    if (!r.ok) break;
    if (m.key == "general.alignment") {
      char* end = nullptr;
      const unsigned long long a = strtoull(m.value.c_str(), &end, 10);
      if (end && *end == '\0' && !m.value.empty() && a >= 1 && a <= 65536 && (a & (a - 1)) == 0)
        g->alignment = a;
      else
        fprintf(stderr, "[aspida_gguf] ignoring invalid general.alignment=%s (keeping 32)\n", m.value.c_str());
    }
    g->meta.push_back(std::move(m));
  }
  for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
    Tensor t;
    t.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok) break;
    if (nd > 4) {
      r.fail("tensor \"" + t.name + "\" has " + std::to_string(nd) + " dims (max 4)");
      break;
    }
    t.n_dims = (int)nd;
    for (uint32_t d = 0; d < nd; ++d) t.dims[d] = r.get<uint64_t>();
    t.ggml_type = (int)r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    uint64_t n = 1;
    for (uint32_t d = 0; d < nd && r.ok; ++d)
      if (!checked_mul(n, t.dims[d], n)) r.fail("tensor \"" + t.name + "\": element count overflows");
    if (r.ok && !byte_size(t.ggml_type, n, t.bytes)) r.fail("tensor \"" + t.name + "\": byte size overflows");
    g->tensors.push_back(std::move(t));
  }
  if (r.ok) {
    g->data_start = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    if (fseek(r.f, 0, SEEK_END) == 0) {
      const long sz = ftell(r.f);
      g->file_size = sz > 0 ? (uint64_t)sz : 0;
    }
    for (const Tensor& t : g->tensors) {
      const uint64_t abs_off = g->data_start + t.offset, end = abs_off + t.bytes;
      if (abs_off < g->data_start || end < abs_off || end > g->file_size) {
        r.fail("tensor \"" + t.name + "\" extends past the end of the file (needs " + std::to_string(end) +
               " bytes, file is " + std::to_string(g->file_size) + ")");
        break;
      }
    }
  }
  fclose(r.f);
  if (!r.ok) {
    g_gguf_err = r.err;
    delete g;
    return nullptr;
  }
  return g;
}

extern "C" const char* aspida_gguf_error(void) { return g_gguf_err.c_str(); }

extern "C" void aspida_gguf_close(aspida_gguf* g) { delete g; }

extern "C" int aspida_gguf_version(const aspida_gguf* g) { return g ? (int)g->version : -EINVAL; }

extern "C" long long aspida_gguf_alignment(const aspida_gguf* g) { return g ? (long long)g->alignment : -EINVAL; }

extern "C" long long aspida_gguf_data_start(const aspida_gguf* g) { return g ? (long long)g->data_start : -EINVAL; }

extern "C" long long aspida_gguf_tensor_count(const aspida_gguf* g) {
  return g ? (long long)g->tensors.size() : -EINVAL;
}

extern "C" long long aspida_gguf_meta_count(const aspida_gguf* g) { return g ? (long long)g->meta.size() : -EINVAL; }

extern "C" const char* aspida_gguf_meta(const aspida_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  for (const Meta& m : g->meta)
    if (m.key == key) return m.value.c_str();
  return nullptr;
}

extern "C" long long aspida_gguf_find(const aspida_gguf* g, const char* name) {
  if (!g || !name) return -EINVAL;
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) return (long long)i;
  return -1;
}

extern "C" int aspida_gguf_tensor(const aspida_gguf* g, long long i, aspida_gguf_tensor_info* out) {
  if (!g || !out || i < 0 || (size_t)i >= g->tensors.size()) return -EINVAL;
  const Tensor& t = g->tensors[(size_t)i];
  out->name = t.name.c_str();
  out->ggml_type = t.ggml_type;
  out->kind = kind_of(t.ggml_type);
  out->n_dims = t.n_dims;
  for (int d = 0; d < 4; ++d) out->dims[d] = (long long)t.dims[d];
  out->file_offset = (long long)(g->data_start + t.offset);
  out->bytes = (long long)t.bytes;
  return 0;
}

extern "C" long long aspida_gguf_read(const aspida_gguf* g, long long i, void* dst, long long cap) {
  if (!g || !dst || i < 0 || (size_t)i >= g->tensors.size()) return -EINVAL;
  const Tensor& t = g->tensors[(size_t)i];
  if (cap < (long long)t.bytes) return -ENOSPC;
  FILE* f = fopen(g->path.c_str(), "rb");
  if (!f) return -errno;
  const bool ok = fseeko(f, (off_t)(g->data_start + t.offset), SEEK_SET) == 0 && fread(dst, 1, t.bytes, f) == t.bytes;
  fclose(f);
  return ok ? (long long)t.bytes : -EIO;
}
