// Converted-snapshot loader: the reference's safetensors container
// (c/st.h, c/qwen.c:2165-2295, 2443-2457, 2330-2346) onto HBM-resident layers.
//
// A snapshot is a directory of *.safetensors files.  Each file is an 8-byte
// little-endian header length, a JSON header {name: {dtype, shape,
// data_offsets}} and the raw data.  MoE tensors, under an optional "model." or
// "model.language_model." prefix:
//   layers.L.mlp.gate.weight                         router, float [E, H]
//   layers.L.mlp.shared_expert_gate.weight           gate row, float [1, H]
//   layers.L.mlp.shared_expert.{gate,up,down}_proj.weight
//   layers.L.mlp.experts.e.{gate,up,down}_proj.weight[.q3|.q2]
// A quantised matrix is a U8/I8 payload [rows, row bytes] with an f32 `.qs`
// [rows, groups] ([rows] for int8) and an optional U8 `.qtype` tag (8, 4, 3,
// 2); without a tag the sizes decide, as load_qmat_mode does.  The `.q3`
// sidecar (c/tools/requantize_expert_q2.py) holds int3 experts with their own
// `.qs` and `.qtype`; it is taken when the caller asks for it (the reference's
// EXPERT_Q3=1, which requires it).  The `.q2` sidecar (EXPERT_Q2=1) holds int2
// experts; an expert without one is read from its main payload, as
// find_qmat_named does (c/qwen.c:2198-2214).
//
// Loading reads tensors with pread into pinned host memory, copies them to a
// device staging buffer and hands them to coli_cuda_moe_layer_set_*, which
// repack the routed experts on the device.  Two staging slots alternate, so
// the file reads of expert e+1 overlap the copy and repack of expert e.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>
#include <dirent.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "sw_backend.h"
#include "sw_moe_layer.h"

using sw::fail_arg;
using sw::fail_hip;

namespace {

enum DType { kBF16 = 0, kF16 = 1, kF32 = 2, kU8 = 3, kI64 = 4 };

struct Tensor {
  int file = -1;
  uint64_t off = 0, nbytes = 0;  // absolute offset of the data in the file
  int dtype = -1;
  std::vector<int64_t> shape;
  int64_t numel = 0;
};

// ---- a JSON reader for safetensors headers --------------------------------
struct Json {
  const char *p, *end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
  }
  bool lit(char c) {
    ws();
    if (p < end && *p == c) {
      p++;
      return true;
    }
    return false;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  bool str(std::string &out) {
    ws();
    if (p >= end || *p != '"') return fail("expected a string");
    p++;
    out.clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end) return fail("bad escape");
        char e = *p++;
        switch (e) {
          case '"': case '\\': case '/': out += e; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (end - p < 4) return fail("bad \\u escape");
            unsigned v = 0;
            for (int i = 0; i < 4; i++) {
              char h = *p++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
              else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
              else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
              else return fail("bad \\u escape");
            }
            // tensor names are ASCII; anything else is kept as UTF-8
            if (v < 0x80) out += (char)v;
            else if (v < 0x800) { out += (char)(0xC0 | (v >> 6)); out += (char)(0x80 | (v & 63)); }
            else { out += (char)(0xE0 | (v >> 12)); out += (char)(0x80 | ((v >> 6) & 63)); out += (char)(0x80 | (v & 63)); }
            break;
          }
          default: return fail("bad escape");
        }
      } else {
        out += c;
      }
    }
    if (p >= end) return fail("unterminated string");
    p++;
    return true;
  }
  bool integer(int64_t &v) {
    ws();
    bool neg = false;
    if (p < end && *p == '-') { neg = true; p++; }
    if (p >= end || *p < '0' || *p > '9') return fail("expected an integer");
    int64_t r = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      if (r > (INT64_MAX - 9) / 10) return fail("integer overflow");
      r = r * 10 + (*p++ - '0');
    }
    v = neg ? -r : r;
    return true;
  }
  // any value, skipped (metadata)
  bool skip(int depth = 0) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    if (*p == '"') { std::string s; return str(s); }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      p++;
      if (lit(close)) return true;
      do {
        if (obj) {
          std::string k;
          if (!str(k) || !lit(':')) return fail("bad object");
        }
        if (!skip(depth + 1)) return false;
      } while (lit(','));
      return lit(close) || fail("bad container");
    }
    while (p < end && *p != ',' && *p != '}' && *p != ']') p++;  // number, true, false, null
    return true;
  }
};

int dtype_code(const std::string &s) {
  if (s == "BF16") return kBF16;
  if (s == "F16") return kF16;
  if (s == "F32") return kF32;
  if (s == "U8" || s == "I8") return kU8;
  if (s == "I64") return kI64;
  return -1;
}
int dtype_size(int d) { return d == kF32 ? 4 : d == kU8 ? 1 : d == kI64 ? 8 : 2; }

float half_to_float(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) bits = s;
    else {  // subnormal: m * 2^-24
      float f = (float)m * 0x1p-24f;
      memcpy(&bits, &f, 4);
      bits |= s;
    }
  } else if (e == 31) {
    bits = s | 0x7F800000u | (m << 13);
  } else {
    bits = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

struct ColiContainer {
  std::vector<std::string> paths;
  std::vector<int> fds;
  std::unordered_map<std::string, Tensor> t;
};

namespace {

bool read_all(int fd, void *dst, size_t bytes, uint64_t off) {
  char *d = (char *)dst;
  while (bytes) {
    const ssize_t r = pread(fd, d, bytes, (off_t)off);
    if (r <= 0) return false;
    d += r;
    bytes -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

int index_file(ColiContainer *c, const std::string &path) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return fail_arg("container: cannot open %s", path.c_str());
  c->paths.push_back(path);
  c->fds.push_back(fd);
  const int fi = (int)c->fds.size() - 1;
  struct stat st;
  if (fstat(fd, &st)) return fail_arg("container: cannot stat %s", path.c_str());
  uint64_t hlen = 0;
  if ((uint64_t)st.st_size < 8 || !read_all(fd, &hlen, 8, 0))
    return fail_arg("container: %s is too short for a safetensors header", path.c_str());
  if (hlen > (512ull << 20) || 8 + hlen > (uint64_t)st.st_size)
    return fail_arg("container: %s declares a %llu-byte header in a %lld-byte file", path.c_str(),
                    (unsigned long long)hlen, (long long)st.st_size);
  std::string hdr(hlen, '\0');
  if (!read_all(fd, &hdr[0], hlen, 8)) return fail_arg("container: cannot read the header of %s", path.c_str());
  const uint64_t data0 = 8 + hlen;
  Json j{hdr.data(), hdr.data() + hdr.size(), {}};
  if (!j.lit('{')) return fail_arg("container: %s: header is not a JSON object", path.c_str());
  if (!j.lit('}')) {
    do {
      std::string name;
      if (!j.str(name) || !j.lit(':')) break;
      if (name == "__metadata__") {
        if (!j.skip()) break;
        continue;
      }
      Tensor t;
      t.file = fi;
      int64_t a = -1, b = -1;
      std::string dt;
      bool have_dt = false, have_off = false, have_shape = false;
      if (!j.lit('{')) { j.fail("tensor entry is not an object"); break; }
      if (!j.lit('}')) {
        do {
          std::string k;
          if (!j.str(k) || !j.lit(':')) break;
          if (k == "dtype") {
            have_dt = j.str(dt);
          } else if (k == "data_offsets") {
            have_off = j.lit('[') && j.integer(a) && j.lit(',') && j.integer(b) && j.lit(']');
          } else if (k == "shape") {
            have_shape = j.lit('[');
            if (have_shape && !j.lit(']')) {
              do {
                int64_t d;
                if (!j.integer(d) || d < 0) { have_shape = false; break; }
                t.shape.push_back(d);
              } while (j.lit(','));
              have_shape = have_shape && j.lit(']');
            }
          } else if (!j.skip()) {
            break;
          }
        } while (j.lit(','));
        if (!j.lit('}')) { j.fail("bad tensor entry"); break; }
      }
      t.dtype = have_dt ? dtype_code(dt) : -1;
      if (!have_dt || !have_off || !have_shape || t.dtype < 0 || a < 0 || b < a)
        return fail_arg("container: %s: tensor '%s' has a malformed or unsupported dtype/shape/data_offsets",
                        path.c_str(), name.c_str());
      t.numel = 1;
      for (int64_t d : t.shape) t.numel *= d;
      t.off = data0 + (uint64_t)a;
      t.nbytes = (uint64_t)(b - a);
      if (t.off + t.nbytes > (uint64_t)st.st_size || (uint64_t)t.numel * dtype_size(t.dtype) != t.nbytes)
        return fail_arg("container: %s: tensor '%s' does not fit its file or its shape", path.c_str(),
                        name.c_str());
      c->t[name] = std::move(t);
    } while (j.lit(','));
    if (!j.err.empty() || !j.lit('}'))
      return fail_arg("container: %s: bad JSON header (%s)", path.c_str(),
                      j.err.empty() ? "unexpected token" : j.err.c_str());
  }
  return 0;
}

const Tensor *find(const ColiContainer *c, const std::string &base, std::string *found = nullptr) {
  static const char *pre[] = {"", "model.", "model.language_model."};
  for (const char *p : pre) {
    auto it = c->t.find(std::string(p) + base);
    if (it != c->t.end()) {
      if (found) *found = it->first;
      return &it->second;
    }
  }
  return nullptr;
}

// A matrix as the reference's load_qmat_mode reads it.
struct QInfo {
  const Tensor *q = nullptr, *s = nullptr;
  int fmt = 0;  // 0 float, 1 int8, 2 int2, 3 int3, 4 int4
  int rows = 0, cols = 0, rb = 0, ng = 0, gs = 0;
};

// sidecar: 0 the main payload, 1 the `.q3` sidecar (required), 2 the `.q2`
// sidecar where there is one, else the main payload
int qinfo(const ColiContainer *c, const std::string &base, int rows, int cols, int sidecar, QInfo &qi) {
  std::string name;
  qi = QInfo();
  qi.rows = rows;
  qi.cols = cols;
  qi.q = find(c, sidecar == 1 ? base + ".q3" : sidecar == 2 ? base + ".q2" : base, &name);
  if (!qi.q && sidecar == 2) qi.q = find(c, base, &name);
  if (!qi.q) return fail_arg("container: missing tensor %s%s", base.c_str(), sidecar == 1 ? ".q3" : "");
  const Tensor &t = *qi.q;
  if (t.dtype != kU8) {
    if (t.dtype == kI64 || t.numel != (int64_t)rows * cols)
      return fail_arg("container: %s: %lld values, expected %d x %d", name.c_str(), (long long)t.numel, rows, cols);
    qi.fmt = 0;
    return 0;
  }
  qi.s = find(c, name + ".qs");
  if (!qi.s || qi.s->dtype == kU8 || qi.s->dtype == kI64)
    return fail_arg("container: quantized tensor %s has no float .qs scales", name.c_str());
  const int64_t ns = qi.s->numel, nb = (int64_t)t.nbytes;
  int qtype = 0;
  if (const Tensor *tt = find(c, name + ".qtype")) {
    unsigned char tag = 0;
    if (tt->numel != 1 || tt->dtype != kU8 || !read_all(c->fds[tt->file], &tag, 1, tt->off))
      return fail_arg("container: %s.qtype is not one U8 tag", name.c_str());
    qtype = tag;
  }
  if (rows <= 0 || nb % rows || ns % rows) return fail_arg("container: %s: payload not divisible into %d rows", name.c_str(), rows);
  qi.rb = (int)(nb / rows);
  qi.ng = (int)(ns / rows);
  if (qtype == 8 || (qtype == 0 && nb == (int64_t)rows * cols && ns == rows)) {
    qi.fmt = 1;
    if (qi.rb != cols) return fail_arg("container: %s: int8 rows of %d bytes, expected %d", name.c_str(), qi.rb, cols);
    // one scale per row (the reference reads only s[row] of an int8 matrix,
    // c/qwen.c:1765-1768); more would not fit the layer's per-row slots
    if (qi.ng != 1)
      return fail_arg("container: %s: int8 matrix with %d scales per row, expected 1", name.c_str(), qi.ng);
  } else if (qtype == 2) {
    qi.fmt = 2;
    qi.gs = qi.ng ? qi.rb * 4 / qi.ng : 0;
  } else if (qtype == 3) {
    qi.fmt = 3;
    if (qi.rb % 3 || !qi.ng) return fail_arg("container: %s: bad int3 packed row", name.c_str());
    qi.gs = (qi.rb / 3 * 8) / qi.ng;
    if (qi.gs <= 0 || qi.gs % 8) return fail_arg("container: %s: bad int3 group geometry", name.c_str());
  } else if (qtype == 0 || qtype == 4) {
    qi.fmt = 4;
    if (!qi.ng) return fail_arg("container: %s: no scales", name.c_str());
    qi.gs = qi.rb * 2 / qi.ng;
    if (qi.gs <= 0) return fail_arg("container: %s: bad int4 group geometry", name.c_str());
  } else {
    return fail_arg("container: %s: unknown qtype tag %d", name.c_str(), qtype);
  }
  if (qi.fmt >= 2 && (int64_t)qi.ng * qi.gs < cols)
    return fail_arg("container: %s: %d groups of %d do not cover %d columns", name.c_str(), qi.ng, qi.gs, cols);
  return 0;
}

// Float tensor (F32 / BF16 / F16) -> f32 host values.
int read_f32(const ColiContainer *c, const Tensor &t, float *dst) {
  if (t.dtype == kF32) return read_all(c->fds[t.file], dst, t.nbytes, t.off) ? 0 : fail_arg("container: read failed");
  if (t.dtype != kBF16 && t.dtype != kF16) return fail_arg("container: tensor is not a float tensor");
  std::vector<uint16_t> raw((size_t)t.numel);
  if (!read_all(c->fds[t.file], raw.data(), t.nbytes, t.off)) return fail_arg("container: read failed");
  for (int64_t i = 0; i < t.numel; i++) {
    if (t.dtype == kBF16) {
      const uint32_t u = (uint32_t)raw[i] << 16;
      memcpy(dst + i, &u, 4);
    } else {
      dst[i] = half_to_float(raw[i]);
    }
  }
  return 0;
}

std::string layer_name(int layer, const char *suffix) { return "layers." + std::to_string(layer) + "." + suffix; }
std::string expert_name(int layer, int e, const char *proj) {
  return layer_name(layer, ("mlp.experts." + std::to_string(e) + "." + proj + ".weight").c_str());
}

// The layer's shape as stored (topk is not part of the container).
int layer_shape(const ColiContainer *c, int layer, int sidecar, ColiMoeShape &s) {
  if (sidecar < 0 || sidecar > 2) return fail_arg("container: sidecar %d (0 main, 1 .q3, 2 .q2)", sidecar);
  const Tensor *r = find(c, layer_name(layer, "mlp.gate.weight"));
  if (!r) return fail_arg("container: layer %d has no router (mlp.gate.weight)", layer);
  if (r->shape.size() != 2 || r->dtype == kU8) return fail_arg("container: layer %d: router is not a float [E, H] matrix", layer);
  const int E = (int)r->shape[0], H = (int)r->shape[1];
  const std::string sgn = layer_name(layer, "mlp.shared_expert.gate_proj.weight");
  const std::string egn = expert_name(layer, 0, "gate_proj") + (sidecar == 1 ? ".q3" : "");
  const Tensor *sg = find(c, sgn), *eg = find(c, egn);
  if (!sg || sg->shape.empty()) return fail_arg("container: missing tensor %s", sgn.c_str());
  if (!eg || eg->shape.empty()) return fail_arg("container: missing tensor %s", egn.c_str());
  const int Ish = (int)sg->shape[0], I = (int)eg->shape[0];
  QInfo gq;
  if (qinfo(c, expert_name(layer, 0, "gate_proj"), I, H, sidecar, gq)) return -1;
  s.hidden = H;
  s.experts = E;
  s.intermediate = I;
  s.shared_intermediate = Ish;
  s.expert_format = gq.fmt;
  s.group_size = gq.gs;
  return 0;
}

struct Pinned {
  void *p = nullptr;
  ~Pinned() {
    if (p) (void)hipHostFree(p);
  }
};
struct DevBuf {
  void *p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

}  // namespace

// ---------------------------------------------------------------------------
extern "C" int coli_cuda_container_open(ColiContainer **out, const char *dir) {
  if (!out || !dir) return fail_arg("coli_cuda_container_open: null argument");
  *out = nullptr;
  DIR *d = opendir(dir);
  if (!d) return fail_arg("coli_cuda_container_open: cannot open directory %s", dir);
  std::vector<std::string> files;
  while (struct dirent *e = readdir(d)) {
    const std::string n = e->d_name;
    if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(std::string(dir) + "/" + n);
  }
  closedir(d);
  if (files.empty()) return fail_arg("coli_cuda_container_open: no .safetensors file in %s", dir);
  std::sort(files.begin(), files.end());
  ColiContainer *c = new ColiContainer();
  for (const std::string &f : files)
    if (index_file(c, f)) {
      for (int fd : c->fds) close(fd);
      delete c;
      return -1;
    }
  *out = c;
  return 0;
}

extern "C" void coli_cuda_container_close(ColiContainer *c) {
  if (!c) return;
  for (int fd : c->fds) close(fd);
  delete c;
}

extern "C" int coli_cuda_container_tensors(const ColiContainer *c) { return c ? (int)c->t.size() : 0; }

extern "C" int coli_cuda_container_moe_shape(const ColiContainer *c, int layer, int sidecar, ColiMoeShape *shape) {
  if (!c || !shape || layer < 0) return fail_arg("coli_cuda_container_moe_shape: invalid argument");
  ColiMoeShape s = *shape;
  if (layer_shape(c, layer, sidecar, s)) return -1;
  *shape = s;
  return 0;
}

extern "C" int coli_cuda_moe_layer_load(ColiCuda *ctx, const ColiContainer *c, int layer, int topk, int sidecar,
                                        ColiMoeLayer **out) {
  if (!ctx || !c || !out || layer < 0 || topk <= 0) return fail_arg("coli_cuda_moe_layer_load: invalid argument");
  *out = nullptr;
  ColiMoeShape s;
  memset(&s, 0, sizeof(s));
  if (layer_shape(c, layer, sidecar, s)) return -1;
  s.topk = topk;
  const int H = s.hidden, E = s.experts, I = s.intermediate, Ish = s.shared_intermediate, fmt = s.expert_format;
  if (fmt < 2 || fmt > 4)
    return fail_arg("coli_cuda_moe_layer_load: layer %d: routed experts are format %d; the device layer takes "
                    "int4, int3 (sidecar 1 for the .q3 sidecar) or int2 (widened to int4 records)", layer, fmt);
  if (s.group_size != 128)
    return fail_arg("coli_cuda_moe_layer_load: layer %d: routed experts in groups of %d; the device layer takes "
                    "groups of 128", layer, s.group_size);
  // the shared expert: int8 rows; router and gate row: float
  QInfo sgq, suq, sdq, gate_row;
  if (qinfo(c, layer_name(layer, "mlp.shared_expert.gate_proj.weight"), Ish, H, 0, sgq) ||
      qinfo(c, layer_name(layer, "mlp.shared_expert.up_proj.weight"), Ish, H, 0, suq) ||
      qinfo(c, layer_name(layer, "mlp.shared_expert.down_proj.weight"), H, Ish, 0, sdq) ||
      qinfo(c, layer_name(layer, "mlp.shared_expert_gate.weight"), 1, H, 0, gate_row))
    return -1;
  if (sgq.fmt != 1 || suq.fmt != 1 || sdq.fmt != 1 || gate_row.fmt != 0)
    return fail_arg("coli_cuda_moe_layer_load: layer %d: the shared expert must be int8 and its gate row float", layer);
  // every routed expert: one format and geometry; int2 and int4 experts may
  // mix (the .q2 sidecar where an expert has one, else its int4 payload), as
  // both are held as int4 records
  std::vector<QInfo> xq((size_t)E * 3);
  static const char *proj[3] = {"gate_proj", "up_proj", "down_proj"};
  const bool mix24 = fmt == 2 || fmt == 4;
  bool any2 = false;
  for (int e = 0; e < E; e++)
    for (int k = 0; k < 3; k++) {
      QInfo &q = xq[(size_t)e * 3 + k];
      if (qinfo(c, expert_name(layer, e, proj[k]), k == 2 ? H : I, k == 2 ? I : H, sidecar, q)) return -1;
      const QInfo &ref = xq[k];
      const bool fmt_ok = q.fmt == fmt || (mix24 && (q.fmt == 2 || q.fmt == 4));
      if (!fmt_ok || q.gs != s.group_size || q.ng != ref.ng || (q.fmt == ref.fmt && q.rb != ref.rb))
        return fail_arg("coli_cuda_moe_layer_load: layer %d expert %d %s: format %d / group %d differs from expert 0",
                        layer, e, proj[k], q.fmt, q.gs);
      const QInfo &g0 = xq[(size_t)e * 3];
      if (k > 0 && q.fmt != g0.fmt)
        return fail_arg("coli_cuda_moe_layer_load: layer %d expert %d: projections in formats %d and %d", layer, e,
                        g0.fmt, q.fmt);
      any2 = any2 || q.fmt == 2;
    }
  if (any2) s.expert_format = 2;
  ColiMoeLayer *L = nullptr;
  if (coli_cuda_moe_layer_create(ctx, &L, &s)) return -1;
  auto bail = [&](int rc) {
    (void)hipStreamSynchronize(ctx->stream);
    coli_cuda_moe_layer_destroy(ctx, L);
    return rc;
  };
  // staging: router + gate row, the shared expert, or one routed expert
  // the largest expert (int4 and int2 experts differ in code bytes)
  size_t expert_b = 0;
  for (int e = 0; e < E; e++) {
    const QInfo *q = &xq[(size_t)e * 3];
    const size_t b = 2 * (q[0].q->nbytes + (size_t)q[0].s->numel * 4) + q[2].q->nbytes + (size_t)q[2].s->numel * 4;
    expert_b = b > expert_b ? b : expert_b;
  }
  const size_t shared_b = 3 * (size_t)Ish * H + (2 * (size_t)Ish + H) * 4;
  const size_t router_b = ((size_t)E + 1) * H * 4;
  const size_t slot = std::max(expert_b, std::max(shared_b, router_b));
  Pinned host[2];
  DevBuf dev[2];
  hipEvent_t done[2] = {nullptr, nullptr};
  for (int i = 0; i < 2; i++) {
    hipError_t e = hipHostMalloc(&host[i].p, slot, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&dev[i].p, slot);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    if (e != hipSuccess) {
      for (hipEvent_t ev : done)
        if (ev) (void)hipEventDestroy(ev);
      fail_hip("coli_cuda_moe_layer_load: staging", e);
      return bail(-1);
    }
  }
  int rc = 0;
  int turn = 0;
  // fill the host slot of this turn (after its previous copy finished), copy
  // it to the device slot and hand it to `use`
  auto stage = [&](auto fill, auto use) -> int {
    char *h = (char *)host[turn].p, *d = (char *)dev[turn].p;
    hipError_t e = hipEventSynchronize(done[turn]);
    if (e != hipSuccess) return fail_hip("coli_cuda_moe_layer_load", e);
    size_t n = 0;
    if (fill(h, n)) return -1;
    e = hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip("coli_cuda_moe_layer_load: upload", e);
    if (use(d)) return -1;
    e = hipEventRecord(done[turn], ctx->stream);
    if (e != hipSuccess) return fail_hip("coli_cuda_moe_layer_load", e);
    turn ^= 1;
    return 0;
  };
  auto raw = [&](const Tensor &t, char *dst) {
    return read_all(c->fds[t.file], dst, t.nbytes, t.off) ? 0 : fail_arg("container: read of %s failed", c->paths[t.file].c_str());
  };
  const Tensor *router = find(c, layer_name(layer, "mlp.gate.weight"));
  rc = stage(
      [&](char *h, size_t &n) {
        n = router_b;
        return read_f32(c, *router, (float *)h) || read_f32(c, *gate_row.q, (float *)(h + (size_t)E * H * 4));
      },
      [&](char *d) {
        return coli_cuda_moe_layer_set_router(ctx, L, (const float *)d, (const float *)(d + (size_t)E * H * 4));
      });
  if (!rc)
    rc = stage(
        [&](char *h, size_t &n) {
          const size_t q = (size_t)Ish * H;
          n = shared_b;
          char *s0 = h + 3 * q;
          return raw(*sgq.q, h) || raw(*suq.q, h + q) || raw(*sdq.q, h + 2 * q) || read_f32(c, *sgq.s, (float *)s0) ||
                 read_f32(c, *suq.s, (float *)(s0 + (size_t)Ish * 4)) ||
                 read_f32(c, *sdq.s, (float *)(s0 + (size_t)Ish * 8));
        },
        [&](char *d) {
          const size_t q = (size_t)Ish * H;
          char *s0 = d + 3 * q;
          return coli_cuda_moe_layer_set_shared_q8(ctx, L, (const signed char *)d, (const float *)s0,
                                                   (const signed char *)(d + q), (const float *)(s0 + (size_t)Ish * 4),
                                                   (const signed char *)(d + 2 * q),
                                                   (const float *)(s0 + (size_t)Ish * 8));
        });
  for (int e = 0; !rc && e < E; e++) {
    const QInfo *q = &xq[(size_t)e * 3];
    const size_t gqb = q[0].q->nbytes, gsb = (size_t)q[0].s->numel * 4, dqb = q[2].q->nbytes;
    rc = stage(
        [&](char *h, size_t &n) {
          n = expert_b;
          char *p = h;
          return raw(*q[0].q, p) || raw(*q[1].q, p + gqb) || read_f32(c, *q[0].s, (float *)(p + 2 * gqb)) ||
                 read_f32(c, *q[1].s, (float *)(p + 2 * gqb + gsb)) || raw(*q[2].q, p + 2 * (gqb + gsb)) ||
                 read_f32(c, *q[2].s, (float *)(p + 2 * (gqb + gsb) + dqb));
        },
        [&](char *d) {
          return sw::set_expert_as(
              ctx, L, e, q[0].fmt, (const unsigned char *)d, (const float *)(d + 2 * gqb),
              (const unsigned char *)(d + gqb), (const float *)(d + 2 * gqb + gsb),
              (const unsigned char *)(d + 2 * (gqb + gsb)), (const float *)(d + 2 * (gqb + gsb) + dqb));
        });
  }
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  for (hipEvent_t ev : done) (void)hipEventDestroy(ev);
  if (!rc && e != hipSuccess) rc = fail_hip("coli_cuda_moe_layer_load", e);
  if (rc) return bail(-1);
  *out = L;
  return 0;
}
