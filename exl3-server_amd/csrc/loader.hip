// EXL3 safetensors loading: the shard header parser and the MoE layer loader.
//
// Reference: src/safetensors.{h,cpp} (header parse, mmap), src/glm5.cpp:284-376
// (load_linear: .trellis/.suh/.svh tensors, the codebook from the .mul1/.mcg marker
// keys, the zero-copy view when (header_len + offset) % 4 == 0, the trellis_pack copy
// otherwise) and glm5.cpp:503-518 (the MoE layer's key names).
//
// Device placement. For every shard the layer reads, one DMA moves the byte range that
// covers the layer's tensors into a device image whose base keeps the file's alignment
// modulo 4 (file byte b lands on an address congruent to b mod 4). A trellis tensor
// whose file position is 4-byte aligned is used in place, as the reference's zero-copy
// view; the others are repacked on the device (k_repack: one aligned output word per
// thread from the two aligned source words that straddle it) into an aligned arena, the
// counterpart of the reference's trellis_pack / unaligned byte path
// (trellis_gemm.cpp:311-316). The small tensors (suh/svh, router, bias, dense weights)
// always get aligned copies. The layer handle owns every buffer.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "exl3_internal.hpp"
#include "exl3_moe.h"

using namespace exl3h;

// ---------------------------------------------------------------------------------
// A minimal JSON reader for safetensors headers: objects, arrays, strings (with
// escapes), integers, and the literals; numbers with fractions are accepted and
// skipped. Only what the header format uses is kept.
// ---------------------------------------------------------------------------------
namespace {

struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  int64_t i = 0;
  bool integral = true;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;
};

struct JParser {
  const char *p, *e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char *what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char *w) {
    const size_t n = std::strlen(w);
    if ((size_t)(e - p) < n || std::memcmp(p, w, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool str(std::string &out) {
    if (p >= e || *p != '"') return fail("expected a string");
    ++p;
    out.clear();
    while (p < e && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= e) return fail("bad escape");
        const char x = *p++;
        switch (x) {
          case '"': c = '"'; break;
          case '\\': c = '\\'; break;
          case '/': c = '/'; break;
          case 'b': c = '\b'; break;
          case 'f': c = '\f'; break;
          case 'n': c = '\n'; break;
          case 'r': c = '\r'; break;
          case 't': c = '\t'; break;
          case 'u': {
            if (e - p < 4) return fail("bad \\u escape");
            unsigned cp = 0;
            for (int k = 0; k < 4; ++k) {
              const char h = *p++;
              cp <<= 4;
              if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
              else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
              else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
              else return fail("bad \\u escape");
            }
            // names are ASCII in practice; other code points are kept as UTF-8
            if (cp < 0x80) {
              out.push_back((char)cp);
            } else if (cp < 0x800) {
              out.push_back((char)(0xC0 | (cp >> 6)));
              out.push_back((char)(0x80 | (cp & 0x3F)));
            } else {
              out.push_back((char)(0xE0 | (cp >> 12)));
              out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
              out.push_back((char)(0x80 | (cp & 0x3F)));
            }
            continue;
          }
          default: return fail("bad escape");
        }
      }
      out.push_back(c);
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool num(JVal &v) {
    const char *s = p;
    if (p < e && (*p == '-' || *p == '+')) ++p;
    bool digits = false;
    int64_t acc = 0;
    bool overflow = false;
    while (p < e && *p >= '0' && *p <= '9') {
      const int d = *p - '0';
      if (acc > (INT64_MAX - d) / 10) overflow = true;
      else acc = acc * 10 + d;
      ++p;
      digits = true;
    }
    if (!digits) return fail("bad number");
    v.kind = JVal::NUM;
    v.i = *s == '-' ? -acc : acc;
    v.integral = !overflow;
    if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) {
      v.integral = false;
      ++p;
      while (p < e && ((*p >= '0' && *p <= '9') || *p == '+' || *p == '-' || *p == 'e' || *p == 'E')) ++p;
    }
    return true;
  }
  bool val(JVal &v, int depth) {
    if (depth > 16) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    const char c = *p;
    if (c == '{') {
      ++p;
      v.kind = JVal::OBJ;
      ws();
      if (p < e && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        v.o.emplace_back(std::move(k), JVal{});
        if (!val(v.o.back().second, depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      v.kind = JVal::ARR;
      ws();
      if (p < e && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        v.a.emplace_back();
        if (!val(v.a.back(), depth + 1)) return false;
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::STR;
      return str(v.s);
    }
    if (c == 't') {
      v.kind = JVal::BOOL;
      v.b = true;
      return lit("true");
    }
    if (c == 'f') {
      v.kind = JVal::BOOL;
      return lit("false");
    }
    if (c == 'n') return lit("null");
    return num(v);
  }
};

const JVal *jget(const JVal &o, const char *k) {
  for (auto &kv : o.o)
    if (kv.first == k) return &kv.second;
  return nullptr;
}

// dtype name -> (exl3_st_dtype, element bytes); the names the reference accepts
// (safetensors.cpp:30-40)
bool dtype_of(const std::string &s, int32_t &dt, int32_t &size) {
  struct D {
    const char *n;
    int32_t dt, sz;
  };
  static const D tab[] = {{"F16", EXL3_ST_F16, 2},  {"BF16", EXL3_ST_BF16, 2}, {"F32", EXL3_ST_F32, 4},
                          {"I16", EXL3_ST_I16, 2},  {"I32", EXL3_ST_I32, 4},   {"U8", EXL3_ST_U8, 1},
                          {"I8", EXL3_ST_I8, 1},    {"I64", EXL3_ST_I64, 8},   {"F64", EXL3_ST_F64, 8},
                          {"U16", EXL3_ST_U16, 2},  {"U32", EXL3_ST_U32, 4},   {"BOOL", EXL3_ST_BOOL, 1}};
  for (const D &d : tab)
    if (s == d.n) {
      dt = d.dt;
      size = d.sz;
      return true;
    }
  return false;
}

}  // namespace

struct exl3_st_file_s {
  std::string path;
  int64_t header_len = 0;  // 8 + JSON length: the data section's file offset
  std::vector<exl3_st_tensor> tensors;
  std::vector<std::string> names;
  std::map<std::string, int> index;
  const uint8_t *map = nullptr;
  size_t map_size = 0;
};

namespace {

void st_unmap(exl3_st_file_s *f) {
  if (f->map) ::munmap((void *)f->map, f->map_size);
  f->map = nullptr;
}

// Repack: dst word w = the 4 bytes at src_base + src_off + 4w, read as the two aligned
// words that straddle them. The source image is padded so that the second word of the
// last output word is inside it.
__global__ __launch_bounds__(256) void k_repack(const uint32_t *__restrict__ src_aligned, uint32_t shift_bytes,
                                                 uint32_t *__restrict__ dst, int64_t words) {
  const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (w >= words) return;
  const uint32_t lo = src_aligned[w], hi = src_aligned[w + 1];
  dst[w] = __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

}  // namespace

extern "C" {

exl3_status exl3_st_open(const char *path, exl3_st_file_t *out) {
  if (!path || !out) return fail(EXL3_ERR_INVALID, "exl3_st_open: null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(EXL3_ERR_INVALID, std::string("cannot open ") + path);
  struct stat sb {};
  if (::fstat(fd, &sb) != 0) {
    ::close(fd);
    return fail(EXL3_ERR_INVALID, std::string("cannot stat ") + path);
  }
  const int64_t size = (int64_t)sb.st_size;
  if (size < 8) {
    ::close(fd);
    return fail(EXL3_ERR_INVALID, std::string("truncated safetensors file ") + path);
  }
  void *base = ::mmap(nullptr, (size_t)size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (base == MAP_FAILED) return fail(EXL3_ERR_INVALID, std::string("mmap failed for ") + path);
  exl3_st_file_s *f = new exl3_st_file_s;
  f->path = path;
  f->map = (const uint8_t *)base;
  f->map_size = (size_t)size;
  uint64_t n = 0;
  std::memcpy(&n, base, 8);  // little-endian u64 header length
  if (n > (uint64_t)(size - 8)) {
    st_unmap(f);
    delete f;
    return fail(EXL3_ERR_INVALID, std::string("invalid safetensors header length in ") + path);
  }
  f->header_len = 8 + (int64_t)n;
  JParser jp{(const char *)base + 8, (const char *)base + 8 + n, {}};
  JVal root;
  if (!jp.val(root, 0) || root.kind != JVal::OBJ) {
    const std::string why = jp.err.empty() ? "not an object" : jp.err;
    st_unmap(f);
    delete f;
    return fail(EXL3_ERR_INVALID, std::string("bad safetensors header in ") + path + ": " + why);
  }
  for (auto &kv : root.o) {
    if (kv.first == "__metadata__") continue;
    const JVal &t = kv.second;
    const JVal *dt = t.kind == JVal::OBJ ? jget(t, "dtype") : nullptr;
    const JVal *sh = t.kind == JVal::OBJ ? jget(t, "shape") : nullptr;
    const JVal *off = t.kind == JVal::OBJ ? jget(t, "data_offsets") : nullptr;
    exl3_st_tensor ti{};
    int32_t esize = 0;
    bool ok = dt && dt->kind == JVal::STR && dtype_of(dt->s, ti.dtype, esize) && sh && sh->kind == JVal::ARR &&
              sh->a.size() <= 8 && off && off->kind == JVal::ARR && off->a.size() == 2;
    int64_t numel = 1;
    if (ok) {
      ti.ndim = (int32_t)sh->a.size();
      for (size_t d = 0; d < sh->a.size() && ok; ++d) {
        const JVal &x = sh->a[d];
        ok = x.kind == JVal::NUM && x.integral && x.i >= 0 && x.i < ((int64_t)1 << 40);
        if (ok) {
          ti.shape[d] = x.i;
          numel = x.i == 0 ? 0 : (numel > ((int64_t)1 << 50) / x.i ? -1 : numel * x.i);
          ok = numel >= 0;
        }
      }
    }
    if (ok) {
      const JVal &a0 = off->a[0], &a1 = off->a[1];
      ok = a0.kind == JVal::NUM && a1.kind == JVal::NUM && a0.integral && a1.integral && a0.i >= 0 && a1.i >= a0.i;
      if (ok) {
        ti.offset = a0.i;
        ti.nbytes = a1.i - a0.i;
        // the reference's consistency check (safetensors.cpp:97)
        ok = ti.nbytes == numel * esize && f->header_len + ti.offset + ti.nbytes <= size;
      }
    }
    if (!ok) {
      st_unmap(f);
      delete f;
      return fail(EXL3_ERR_INVALID, "bad or inconsistent entry for tensor " + kv.first + " in " + path);
    }
    ti.file_offset = f->header_len + ti.offset;
    f->index[kv.first] = (int)f->tensors.size();
    f->tensors.push_back(ti);
    f->names.push_back(kv.first);
  }
  *out = f;
  return EXL3_OK;
}

exl3_status exl3_st_close(exl3_st_file_t f) {
  if (!f) return EXL3_OK;
  st_unmap(f);
  delete f;
  return EXL3_OK;
}

int64_t exl3_st_header_len(exl3_st_file_t f) { return f ? f->header_len : -1; }

int32_t exl3_st_count(exl3_st_file_t f) { return f ? (int32_t)f->tensors.size() : 0; }

exl3_status exl3_st_tensor_at(exl3_st_file_t f, int32_t i, exl3_st_tensor *info, const char **name) {
  if (!f || !info || i < 0 || i >= (int32_t)f->tensors.size())
    return fail(EXL3_ERR_INVALID, "exl3_st_tensor_at: bad arguments");
  *info = f->tensors[(size_t)i];
  if (name) *name = f->names[(size_t)i].c_str();
  return EXL3_OK;
}

exl3_status exl3_st_find(exl3_st_file_t f, const char *name, exl3_st_tensor *info) {
  if (!f || !name || !info) return fail(EXL3_ERR_INVALID, "exl3_st_find: null argument");
  auto it = f->index.find(name);
  if (it == f->index.end()) return fail(EXL3_ERR_INVALID, std::string("no tensor ") + name + " in " + f->path);
  *info = f->tensors[(size_t)it->second];
  return EXL3_OK;
}

const void *exl3_st_data(exl3_st_file_t f, const char *name) {
  if (!f || !name) return nullptr;
  auto it = f->index.find(name);
  if (it == f->index.end()) return nullptr;
  return f->map + f->tensors[(size_t)it->second].file_offset;
}

}  // extern "C"

// ---------------------------------------------------------------------------------
// The MoE layer loader
// ---------------------------------------------------------------------------------
namespace {

struct Src {
  exl3_st_file_s *f = nullptr;
  exl3_st_tensor t{};
  bool ok = false;
};

struct Loader {
  std::vector<exl3_st_file_s *> files;
  std::vector<void *> owned;  // device buffers (handed to the layer on success)
  hipStream_t st = nullptr;

  ~Loader() {
    for (void *p : owned) (void)hipFree(p);
  }
  Src find(const std::string &name) const {
    Src s;
    for (auto *f : files) {
      auto it = f->index.find(name);
      if (it != f->index.end()) {
        s.f = f;
        s.t = f->tensors[(size_t)it->second];
        s.ok = true;
        return s;
      }
    }
    return s;
  }
  exl3_status dev_alloc(size_t bytes, void **p) {
    *p = nullptr;
    EXL3_HIP(hipMalloc(p, bytes));
    owned.push_back(*p);
    return EXL3_OK;
  }
};

struct Need {
  std::string name;
  Src src;
  bool trellis;
  void **dst;  // where the device pointer goes
};

}  // namespace

extern "C" {

exl3_status exl3_moe_layer_load(const char *const *shard_paths, int32_t n_shards, const char *prefix,
                                const exl3_moe_config *cfg, exl3_moe_layer_t *out_layer,
                                exl3_stream_t stream) {
  if (!shard_paths || n_shards <= 0 || !prefix || !cfg || !out_layer)
    return fail(EXL3_ERR_INVALID, "exl3_moe_layer_load: bad arguments");
  *out_layer = nullptr;
  const int E = cfg->n_routed_experts, H = cfg->hidden_size;
  if (E <= 0 || H <= 0) return fail(EXL3_ERR_INVALID, "exl3_moe_layer_load: bad config");
  Loader L;
  L.st = stream_of(stream);
  struct Closer {
    Loader &l;
    ~Closer() {
      for (auto *f : l.files) exl3_st_close(f);
    }
  } closer{L};
  for (int i = 0; i < n_shards; ++i) {
    exl3_st_file_t f = nullptr;
    exl3_status rc = exl3_st_open(shard_paths[i], &f);
    if (rc) return rc;
    L.files.push_back(f);
  }
  const std::string m(prefix);

  // linear descriptors in the reference's order: experts e*3 + {gate, up, down}
  // (glm5.cpp:511-517), then the shared expert's three
  std::vector<exl3_linear_desc> experts((size_t)E * 3), shared(3);
  bool have_shared = false;
  std::vector<Need> needs;
  std::vector<std::pair<Src, exl3_linear_desc *>> dense_lin;  // plain .weight linears
  auto add_linear = [&](const std::string &key, exl3_linear_desc &d) -> exl3_status {
    std::memset(&d, 0, sizeof(d));
    const Src tr = L.find(key + ".trellis");
    if (tr.ok) {
      if (tr.t.ndim != 3 || tr.t.dtype != EXL3_ST_I16 || tr.t.shape[2] % 16 != 0)
        return fail(EXL3_ERR_INVALID, key + ".trellis must be an (in/16, out/16, 16K) int16 array");
      d.tw.K = (int32_t)(tr.t.shape[2] / 16);
      // the codebook from the marker keys (glm5.cpp:303)
      d.tw.codebook = L.find(key + ".mul1").ok ? EXL3_CB_MUL1 : (L.find(key + ".mcg").ok ? EXL3_CB_MCG : EXL3_CB_3INST);
      d.in_features = d.tw.in_features = (int32_t)(tr.t.shape[0] * 16);
      d.out_features = d.tw.out_features = (int32_t)(tr.t.shape[1] * 16);
      const Src su = L.find(key + ".suh"), sv = L.find(key + ".svh");
      if (!su.ok || !sv.ok || su.t.dtype != EXL3_ST_F16 || sv.t.dtype != EXL3_ST_F16 ||
          su.t.nbytes != 2 * (int64_t)d.in_features || sv.t.nbytes != 2 * (int64_t)d.out_features)
        return fail(EXL3_ERR_INVALID, key + ": missing or malformed .suh/.svh");
      needs.push_back({key + ".trellis", tr, true, (void **)&d.tw.trellis});
      needs.push_back({key + ".suh", su, false, (void **)&d.tw.suh});
      needs.push_back({key + ".svh", sv, false, (void **)&d.tw.svh});
      return EXL3_OK;
    }
    const Src w = L.find(key + ".weight");
    if (w.ok) {
      if (w.t.ndim != 2 || w.t.dtype != EXL3_ST_F16)
        return fail(EXL3_ERR_UNSUPPORTED, key + ".weight: only 2-D f16 dense weights are loaded");
      // stored (out, in) as in the checkpoint; the descriptor takes (in, out)
      d.out_features = (int32_t)w.t.shape[0];
      d.in_features = (int32_t)w.t.shape[1];
      dense_lin.push_back({w, &d});
      return EXL3_OK;
    }
    return fail(EXL3_ERR_INVALID, "missing linear " + key);
  };
  static const char *kProj[3] = {"gate_proj", "up_proj", "down_proj"};
  for (int e = 0; e < E; ++e)
    for (int j = 0; j < 3; ++j) {
      exl3_status rc = add_linear(m + "experts." + std::to_string(e) + "." + kProj[j], experts[(size_t)(e * 3 + j)]);
      if (rc) return rc;
    }
  if (L.find(m + "shared_experts.gate_proj.trellis").ok || L.find(m + "shared_experts.gate_proj.weight").ok) {
    have_shared = true;
    for (int j = 0; j < 3; ++j) {
      exl3_status rc = add_linear(m + "shared_experts." + kProj[j], shared[(size_t)j]);
      if (rc) return rc;
    }
  }
  const Src rw = L.find(m + "gate.weight"), rb = L.find(m + "gate.e_score_correction_bias");
  if (!rw.ok || rw.t.ndim != 2 || rw.t.dtype != EXL3_ST_F16 || rw.t.shape[0] != E || rw.t.shape[1] != H)
    return fail(EXL3_ERR_INVALID, m + "gate.weight must be an (E, hidden) f16 array");
  if (!rb.ok || rb.t.dtype != EXL3_ST_F32 || rb.t.nbytes != 4 * (int64_t)E)
    return fail(EXL3_ERR_INVALID, m + "gate.e_score_correction_bias must be an (E) f32 array");
  const void *router_w = nullptr, *router_b = nullptr;
  needs.push_back({m + "gate.weight", rw, false, (void **)&router_w});
  needs.push_back({m + "gate.e_score_correction_bias", rb, false, (void **)&router_b});
  for (const Need &n : needs)
    if (n.src.t.nbytes % 4 != 0) return fail(EXL3_ERR_UNSUPPORTED, n.name + ": size not a multiple of 4 bytes");

  // one device image per shard: the byte range covering the layer's tensors, placed so
  // that file byte b sits on an address congruent to b mod 4, plus 8 bytes of padding
  // for the repack kernel's straddling reads
  std::map<exl3_st_file_s *, std::pair<int64_t, int64_t>> range;  // file -> [lo, hi)
  for (const Need &n : needs) {
    auto &r = range.emplace(n.src.f, std::make_pair(INT64_MAX, (int64_t)0)).first->second;
    r.first = std::min(r.first, n.src.t.file_offset);
    r.second = std::max(r.second, n.src.t.file_offset + n.src.t.nbytes);
  }
  std::map<exl3_st_file_s *, uint8_t *> image;  // device address of file byte `lo`
  for (auto &kv : range) {
    const int64_t lo = kv.second.first, hi = kv.second.second;
    void *buf = nullptr;
    exl3_status rc = L.dev_alloc((size_t)(hi - lo) + 16, &buf);
    if (rc) return rc;
    uint8_t *at = (uint8_t *)buf + (lo % 4);  // buf is 256-aligned
    EXL3_HIP(hipMemcpyAsync(at, kv.first->map + lo, (size_t)(hi - lo), hipMemcpyHostToDevice, L.st));
    image[kv.first] = at;
  }
  // the aligned arena: every tensor that is not used in place (256-byte slots)
  size_t arena_bytes = 0;
  auto in_place = [](const Need &n) { return n.trellis && n.src.t.file_offset % 4 == 0; };
  for (const Need &n : needs)
    if (!in_place(n)) arena_bytes += align_up((size_t)n.src.t.nbytes, 256);
  uint8_t *arena = nullptr;
  if (arena_bytes) {
    void *p = nullptr;
    exl3_status rc = L.dev_alloc(arena_bytes, &p);
    if (rc) return rc;
    arena = (uint8_t *)p;
  }
  size_t at = 0;
  int64_t repacked_trellis = 0, in_place_trellis = 0;
  for (const Need &n : needs) {
    uint8_t *src = image[n.src.f] + (n.src.t.file_offset - range[n.src.f].first);
    if (in_place(n)) {
      *n.dst = src;
      ++in_place_trellis;
      continue;
    }
    uint8_t *dst = arena + at;
    at += align_up((size_t)n.src.t.nbytes, 256);
    const uintptr_t sa = (uintptr_t)src;
    const int64_t words = n.src.t.nbytes / 4;
    if (words > 0) {
      k_repack<<<(unsigned)((words + 255) / 256), 256, 0, L.st>>>((const uint32_t *)(sa & ~(uintptr_t)3),
                                                                   (uint32_t)(sa & 3), (uint32_t *)dst, words);
      EXL3_LAUNCHED("k_repack");
    }
    if (n.trellis) ++repacked_trellis;
    *n.dst = dst;
  }
  // dense linears: (out, in) in the file, (in, out) in the descriptor, transposed on
  // the host once at load
  for (auto &dl : dense_lin) {
    const int in = dl.second->in_features, out = dl.second->out_features;
    const uint16_t *w = (const uint16_t *)(dl.first.f->map + dl.first.t.file_offset);
    std::vector<uint16_t> t((size_t)in * out);
    for (int o = 0; o < out; ++o)
      for (int i = 0; i < in; ++i) t[(size_t)i * out + o] = w[(size_t)o * in + i];
    void *p = nullptr;
    exl3_status rc = L.dev_alloc(t.size() * 2, &p);
    if (rc) return rc;
    EXL3_HIP(hipMemcpyAsync(p, t.data(), t.size() * 2, hipMemcpyHostToDevice, L.st));
    EXL3_HIP(hipStreamSynchronize(L.st));  // t leaves scope
    dl.second->dense = (const uint16_t *)p;
  }
  EXL3_HIP(hipStreamSynchronize(L.st));

  exl3_moe_layer_desc desc{};
  desc.experts = experts.data();
  desc.shared = have_shared ? shared.data() : nullptr;
  desc.router_w = (const uint16_t *)router_w;
  desc.router_bias = (const float *)router_b;
  exl3_moe_layer_t layer = nullptr;
  exl3_status rc = exl3_moe_layer_create(&desc, cfg, &layer);
  if (rc) return rc;
  layer_adopt(layer, L.owned, in_place_trellis, repacked_trellis);
  L.owned.clear();
  *out_layer = layer;
  return EXL3_OK;
}


}  // extern "C"

// ---------------------------------------------------------------------------------
// The MLP sub-block's own tensors (post_attention_layernorm, hc_ffn_*)
// ---------------------------------------------------------------------------------
namespace {

// IEEE round to nearest, ties to even, double -> f16 bits (overflow to inf, NaN to the
// quiet NaN 0x7e00): the conversion the reference's load_any applies to F32 and BF16
// tensors (glm5.cpp:236-238, fp16.h:26-63).
uint16_t f16_bits_rne(double x) {
  if (std::isnan(x)) return 0x7e00;
  const uint16_t sign = std::signbit(x) ? 0x8000 : 0x0000;
  const double m = std::fabs(x);
  if (m == 0.0) return sign;
  if (std::isinf(m)) return sign | 0x7c00;
  int e = 0;
  const double fr = std::frexp(m, &e);  // m = fr * 2^e, fr in [0.5, 1)
  if (e >= -13) {  // normal range: m >= 2^-14
    double r = std::nearbyint(std::ldexp(fr, 11));  // 11 significant bits, [1024, 2048]
    int ex = e + 14;
    if (r >= 2048.0) {
      r = 1024.0;
      ex += 1;
    }
    if (ex > 30) return sign | 0x7c00;
    return (uint16_t)(sign | (ex << 10) | ((uint32_t)r - 1024u));
  }
  const double r = std::nearbyint(std::ldexp(m, 24));  // subnormal: units of 2^-24
  return (uint16_t)(sign | (r >= 1024.0 ? 0x0400u : (uint32_t)r));
}

double f16_bits_to_double(uint16_t h) {
  const int s = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  double v = e == 0 ? std::ldexp((double)m, -24)
                    : e == 31 ? (m ? NAN : INFINITY) : std::ldexp(1.0 + m / 1024.0, e - 15);
  return s ? -v : v;
}

// bf16 -> f16 bits: widened to f32 (exact), then one RNE (fp16.h:70-75)
uint16_t f16_from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f16_bits_rne((double)f);
}

// One tensor as load_any reads it (glm5.cpp:205-281): `n` elements to f16 bits or to f32.
exl3_status tensor_as(const Src &s, const std::string &name, int64_t n, std::vector<uint16_t> *h16,
                      std::vector<float> *h32) {
  int64_t numel = 1;
  for (int i = 0; i < s.t.ndim; ++i) numel *= s.t.shape[i];
  if (numel != n) return fail(EXL3_ERR_INVALID, name + ": expected " + std::to_string(n) + " elements");
  const uint8_t *src = s.f->map + s.t.file_offset;
  if (s.t.dtype != EXL3_ST_F16 && s.t.dtype != EXL3_ST_BF16 && s.t.dtype != EXL3_ST_F32)
    return fail(EXL3_ERR_UNSUPPORTED, name + ": only F16, BF16 and F32 tensors are converted");
  auto f16_at = [&](int64_t i) -> uint16_t {
    uint16_t v16;
    float v32;
    switch (s.t.dtype) {
      case EXL3_ST_F16: std::memcpy(&v16, src + 2 * i, 2); return v16;
      case EXL3_ST_BF16: std::memcpy(&v16, src + 2 * i, 2); return f16_from_bf16(v16);
      default: std::memcpy(&v32, src + 4 * i, 4); return f16_bits_rne((double)v32);
    }
  };
  if (h16) {
    h16->resize((size_t)n);
    for (int64_t i = 0; i < n; ++i) (*h16)[(size_t)i] = f16_at(i);
  } else {
    h32->resize((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
      if (s.t.dtype == EXL3_ST_F32) {
        std::memcpy(&(*h32)[(size_t)i], src + 4 * i, 4);
      } else {
        // F16 widened; BF16 through its f16 value, as the reference does for f32 requests
        (*h32)[(size_t)i] = (float)f16_bits_to_double(f16_at(i));
      }
    }
  }
  return EXL3_OK;
}

}  // namespace

extern "C" {

exl3_status exl3_moe_layer_load_block(exl3_moe_layer_t layer, const char *const *shard_paths, int32_t n_shards,
                                      const char *layer_prefix, exl3_hc_site *site, const uint16_t **norm_w,
                                      exl3_stream_t stream) {
  if (!layer || !shard_paths || n_shards <= 0 || !layer_prefix || !site || !norm_w)
    return fail(EXL3_ERR_INVALID, "exl3_moe_layer_load_block: bad arguments");
  const int N = site->mult, D = layer_hidden(layer);
  if (N < 1 || N > 8) return fail(EXL3_ERR_UNSUPPORTED, "hc_mult must be 1..8");
  Loader L;
  L.st = stream_of(stream);
  struct Closer {
    Loader &l;
    ~Closer() {
      for (auto *f : l.files) exl3_st_close(f);
    }
  } closer{L};
  for (int i = 0; i < n_shards; ++i) {
    exl3_st_file_t f = nullptr;
    exl3_status rc = exl3_st_open(shard_paths[i], &f);
    if (rc) return rc;
    L.files.push_back(f);
  }
  const std::string lp(layer_prefix);
  const int W = (2 + N) * N;
  const char *keys[4] = {"post_attention_layernorm.weight", "hc_ffn_fn", "hc_ffn_base", "hc_ffn_scale"};
  Src src[4];
  for (int i = 0; i < 4; ++i) {
    src[i] = L.find(lp + keys[i]);
    if (!src[i].ok) return fail(EXL3_ERR_INVALID, "missing tensor " + lp + keys[i]);
  }
  if (src[1].t.ndim != 2 || src[1].t.shape[0] != W || src[1].t.shape[1] != (int64_t)N * D)
    return fail(EXL3_ERR_INVALID, lp + "hc_ffn_fn must be ((2 + mult) * mult, mult * hidden)");
  std::vector<uint16_t> nw;
  std::vector<float> fn, base, scale;
  exl3_status rc = tensor_as(src[0], lp + keys[0], D, &nw, nullptr);
  if (!rc) rc = tensor_as(src[1], lp + keys[1], (int64_t)W * N * D, nullptr, &fn);
  if (!rc) rc = tensor_as(src[2], lp + keys[2], W, nullptr, &base);
  if (!rc) rc = tensor_as(src[3], lp + keys[3], 3, nullptr, &scale);
  if (rc) return rc;
  // one buffer: fn (16-byte aligned, as exl3_hc_prepare requires), base, scale, norm weight
  const size_t o_fn = 0, o_base = align_up(fn.size() * 4, 256), o_scale = o_base + align_up(base.size() * 4, 256);
  const size_t o_nw = o_scale + 256, total = o_nw + align_up(nw.size() * 2, 256);
  void *buf = nullptr;
  rc = L.dev_alloc(total, &buf);
  if (rc) return rc;
  uint8_t *b = (uint8_t *)buf;
  EXL3_HIP(hipMemcpyAsync(b + o_fn, fn.data(), fn.size() * 4, hipMemcpyHostToDevice, L.st));
  EXL3_HIP(hipMemcpyAsync(b + o_base, base.data(), base.size() * 4, hipMemcpyHostToDevice, L.st));
  EXL3_HIP(hipMemcpyAsync(b + o_scale, scale.data(), scale.size() * 4, hipMemcpyHostToDevice, L.st));
  EXL3_HIP(hipMemcpyAsync(b + o_nw, nw.data(), nw.size() * 2, hipMemcpyHostToDevice, L.st));
  EXL3_HIP(hipStreamSynchronize(L.st));  // the host vectors leave scope
  layer_adopt(layer, L.owned, 0, 0);
  L.owned.clear();
  site->fn = (const float *)(b + o_fn);
  site->base = (const float *)(b + o_base);
  site->scale = (const float *)(b + o_scale);
  *norm_w = (const uint16_t *)(b + o_nw);
  return EXL3_OK;
}

}  // extern "C"
