// fgpt_weights.hip -- host-side file reading: checkpoints for
// fg_weights_read, and eval rows for fg_rows_npy. Checkpoints are
// the two on-disk formats load_gpt_weights accepts
// (src/lib/load_weights.f90:830-874): model.safetensors with canonical names
// and arch.* metadata (:446-592), or one 1-D <f4 .npy file per tensor
// (:139-169, :853-873) with an optional arch.txt (require_arch,
// src/lib/fortran_arch.f90:238-246). No device code.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/fgpt.h"
#include "fgpt_internal.h"

namespace fgpt {
namespace {

int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t fail(int32_t code, const char* fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  return set_error(code, msg);
}

#define TRY(x)                  \
  do {                          \
    int32_t r_ = (x);           \
    if (r_ != FG_OK) return r_; \
  } while (0)

bool file_exists(const std::string& p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

// ------------------------------------------------------------------ .npy
// version 1/2/3 header, dtype '<f4', C order, 1-D, exactly `want` values
int32_t read_npy_f32(const std::string& path, size_t want, float* dst) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return fail(FG_EWEIGHT, "load failed (missing file): %s", path.c_str());
  unsigned char mg[8];
  int32_t rc = FG_OK;
  std::string hdr;
  uint32_t hlen = 0;
  if (fread(mg, 1, 8, f) != 8 || memcmp(mg, "\x93NUMPY", 6) != 0) {
    rc = fail(FG_EWEIGHT, "not a .npy file (missing or empty): %s", path.c_str());
  } else {
    if (mg[6] == 1) {
      unsigned char b[2];
      if (fread(b, 1, 2, f) != 2) rc = fail(FG_EWEIGHT, "truncated header: %s", path.c_str());
      hlen = b[0] | (b[1] << 8);
    } else {
      unsigned char b[4];
      if (fread(b, 1, 4, f) != 4) rc = fail(FG_EWEIGHT, "truncated header: %s", path.c_str());
      hlen = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
    }
    if (rc == FG_OK) {
      hdr.resize(hlen);
      if (hlen > 65536 || fread(&hdr[0], 1, hlen, f) != hlen)
        rc = fail(FG_EWEIGHT, "truncated header: %s", path.c_str());
    }
  }
  if (rc == FG_OK) {
    auto has = [&](const char* s) { return hdr.find(s) != std::string::npos; };
    if (!has("'descr': '<f4'"))
      rc = fail(FG_EWEIGHT, "%s: dtype is not '<f4'", path.c_str());
    else if (!has("'fortran_order': False"))
      rc = fail(FG_EWEIGHT, "%s: fortran_order arrays are not supported", path.c_str());
    else {
      size_t p = hdr.find("'shape': (");
      unsigned long long n = 0;
      char tail = 0;
      if (p == std::string::npos ||
          sscanf(hdr.c_str() + p + 10, "%llu%c", &n, &tail) != 2 || tail != ',')
        rc = fail(FG_EWEIGHT, "%s: shape is not 1-D", path.c_str());
      else if (hdr.find(')', p) < hdr.find(',', p) ||
               hdr.find(',', hdr.find(',', p) + 1) < hdr.find(')', p))
        rc = fail(FG_EWEIGHT, "%s: shape is not 1-D", path.c_str());
      else if (n != want)
        rc = fail(FG_EWEIGHT, "%s: %llu values, expected %zu", path.c_str(), n, want);
      else if (fread(dst, 4, want, f) != want)
        rc = fail(FG_EWEIGHT, "%s: truncated payload", path.c_str());
    }
  }
  fclose(f);
  return rc;
}

int32_t check_arch_txt(const std::string& dir, const Dims& d) {
  FILE* f = fopen((dir + "/arch.txt").c_str(), "r");
  if (!f) return FG_OK;  // absent = accepted, as read_arch_txt does
  char line[256];
  int32_t rc = FG_OK;
  while (fgets(line, sizeof line, f)) {
    if (line[0] == '#') continue;
    char key[64];
    long val;
    if (sscanf(line, " %63[a-z_] = %ld", key, &val) != 2) continue;
    long want = -1;
    if (!strcmp(key, "d_model")) want = d.D;
    else if (!strcmp(key, "n_head")) want = d.H;
    else if (!strcmp(key, "n_kv")) want = d.KH;
    else if (!strcmp(key, "n_layer")) want = d.L;
    else if (!strcmp(key, "vocab")) want = d.V;
    else if (!strcmp(key, "head_dim")) want = d.hd;
    if (want >= 0 && want != val) {
      rc = fail(FG_EARCH, "arch.txt %s = %ld but the dims say %ld", key, val, want);
      break;
    }
  }
  fclose(f);
  return rc;
}

// ------------------------------------------------------------ safetensors
// File: u64 LE header length n, n bytes of JSON, then the data buffer.
// Header: {"NAME": {"dtype": "F32", "shape": [..], "data_offsets": [b, e]},
// ..., "__metadata__": {"key": "value", ...}}; offsets are relative to the
// data buffer.
struct StEntry {
  std::string dtype;
  std::vector<uint64_t> shape;
  uint64_t begin = 0, end = 0;
};

struct StFile {
  std::map<std::string, StEntry> tensors;
  std::map<std::string, std::string> meta;
  uint64_t data0 = 0, size = 0;
};

// A JSON reader for exactly that header grammar (strings, non-negative
// integers, arrays of them, objects); any other token is a format error.
struct Json {
  const std::string& s;
  size_t i = 0;
  bool ok = true;
  explicit Json(const std::string& t) : s(t) {}
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
  }
  bool eat(char c) {
    ws();
    if (i < s.size() && s[i] == c) {
      ++i;
      return true;
    }
    return false;
  }
  bool peek(char c) {
    ws();
    return i < s.size() && s[i] == c;
  }
  std::string str() {
    std::string out;
    if (!eat('"')) {
      ok = false;
      return out;
    }
    while (i < s.size() && s[i] != '"') {
      char c = s[i++];
      if (c == '\\' && i < s.size()) {
        const char e = s[i++];
        if (e == 'n') c = '\n';
        else if (e == 't') c = '\t';
        else if (e == 'r') c = '\r';
        else if (e == 'b') c = '\b';
        else if (e == 'f') c = '\f';
        else if (e == 'u') {  // \uXXXX: keep ASCII, reject the rest
          unsigned v = 0;
          if (i + 4 > s.size() || sscanf(s.c_str() + i, "%4x", &v) != 1 || v > 0x7f) ok = false;
          i += 4;
          c = (char)v;
        } else c = e;
      }
      out += c;
    }
    if (!eat('"')) ok = false;
    return out;
  }
  uint64_t num() {
    ws();
    uint64_t v = 0;
    size_t j = i;
    while (i < s.size() && s[i] >= '0' && s[i] <= '9') v = v * 10 + (uint64_t)(s[i++] - '0');
    if (i == j) ok = false;
    return v;
  }
  std::vector<uint64_t> nums() {
    std::vector<uint64_t> v;
    if (!eat('[')) {
      ok = false;
      return v;
    }
    if (eat(']')) return v;
    do v.push_back(num());
    while (ok && eat(','));
    if (!eat(']')) ok = false;
    return v;
  }
};

int32_t st_open(const std::string& path, StFile* out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return fail(FG_EWEIGHT, "cannot open %s", path.c_str());
  fseek(f, 0, SEEK_END);
  const long fsz = ftell(f);
  fseek(f, 0, SEEK_SET);
  unsigned char b[8];
  if (fsz < 8 || fread(b, 1, 8, f) != 8) {
    fclose(f);
    return fail(FG_EWEIGHT, "%s: not a safetensors file (too short)", path.c_str());
  }
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | b[k];
  if (n == 0 || n > (uint64_t)fsz - 8 || n > (100u << 20)) {
    fclose(f);
    return fail(FG_EWEIGHT, "%s: bad header length %llu", path.c_str(), (unsigned long long)n);
  }
  std::string hdr(n, '\0');
  const size_t got = fread(&hdr[0], 1, n, f);
  fclose(f);
  if (got != n) return fail(FG_EWEIGHT, "%s: truncated header", path.c_str());
  Json j(hdr);
  if (!j.eat('{')) return fail(FG_EWEIGHT, "%s: header is not a JSON object", path.c_str());
  if (!j.eat('}')) {
    do {
      const std::string key = j.str();
      if (!j.ok || !j.eat(':')) break;
      if (key == "__metadata__") {
        if (!j.eat('{')) {
          j.ok = false;
          break;
        }
        if (!j.eat('}')) {
          do {
            const std::string mk = j.str();
            if (!j.ok || !j.eat(':')) {
              j.ok = false;
              break;
            }
            out->meta[mk] = j.str();
          } while (j.ok && j.eat(','));
          if (!j.eat('}')) j.ok = false;
        }
      } else {
        StEntry e;
        bool have_off = false;
        if (!j.eat('{')) {
          j.ok = false;
          break;
        }
        do {
          const std::string f2 = j.str();
          if (!j.ok || !j.eat(':')) {
            j.ok = false;
            break;
          }
          if (f2 == "dtype") {
            e.dtype = j.str();
          } else if (f2 == "shape") {
            e.shape = j.nums();
          } else if (f2 == "data_offsets") {
            const std::vector<uint64_t> o = j.nums();
            if (o.size() != 2) j.ok = false;
            else {
              e.begin = o[0];
              e.end = o[1];
              have_off = true;
            }
          } else {
            j.ok = false;
          }
        } while (j.ok && j.eat(','));
        if (!j.eat('}') || !have_off) j.ok = false;
        out->tensors[key] = e;
      }
    } while (j.ok && j.eat(','));
    if (j.ok && !j.eat('}')) j.ok = false;
  }
  if (!j.ok) return fail(FG_EWEIGHT, "%s: malformed header near byte %zu", path.c_str(), j.i);
  out->data0 = 8 + n;
  out->size = (uint64_t)fsz;
  return FG_OK;
}

// arch_canonical_of / arch_id_of (src/lib/fortran_arch.f90:200-236): the
// canonical JSON of the eight fields and its 64-bit rotate-xor digest.
std::string arch_canonical(long d, long nh, long nkv, long hd, long nl, long vv, long ctx,
                           long bos) {
  char buf[320];
  snprintf(buf, sizeof buf,
           "{\"schema\":\"fortran_gpt/arch/1\",\"d_model\":%ld,\"n_head\":%ld,\"n_kv\":%ld,"
           "\"head_dim\":%ld,\"n_layer\":%ld,\"vocab\":%ld,\"ctx\":%ld,\"bos\":%ld}",
           d, nh, nkv, hd, nl, vv, ctx, bos);
  return buf;
}

std::string arch_id(const std::string& s) {
  uint64_t acc = 0x0123456789abcdefull;
  for (unsigned char c : s) {
    acc ^= c;
    acc = (acc << 17) | (acc >> 47);
    acc ^= acc >> 29;
  }
  char hex[17];
  snprintf(hex, sizeof hex, "%016llx", (unsigned long long)acc);
  return hex;
}

// a metadata integer: absent -> false; present but not an integer -> error
int32_t meta_int(const StFile& st, const std::string& path, const char* key, long* val,
                 bool* found) {
  *found = false;
  auto it = st.meta.find(key);
  if (it == st.meta.end()) return FG_OK;
  const char* p = it->second.c_str();
  char* endp = nullptr;
  const long v = strtol(p, &endp, 10);
  while (endp && *endp == ' ') ++endp;
  if (endp == p || !endp || *endp != '\0')
    return fail(FG_EARCH, "metadata %s in %s is not an integer: \"%s\"", key, path.c_str(), p);
  *val = v;
  *found = true;
  return FG_OK;
}

// check_declared_arch + check_arch_selfconsistent (load_weights.f90:533-590)
int32_t st_check_arch(const StFile& st, const std::string& path, const Dims& d) {
  const struct {
    const char* key;
    long want;
  } fields[] = {{"arch.d_model", d.D}, {"arch.n_head", d.H},     {"arch.n_kv", d.KH},
                {"arch.n_layer", d.L}, {"arch.vocab", d.V},      {"arch.head_dim", d.hd}};
  for (const auto& f : fields) {
    long v = 0;
    bool found = false;
    TRY(meta_int(st, path, f.key, &v, &found));
    if (found && v != f.want)
      return fail(FG_EARCH, "architecture mismatch (%s): the dims say %ld, %s declares %ld", f.key,
                  f.want, path.c_str(), v);
  }
  const char* keys[8] = {"arch.d_model", "arch.n_head", "arch.n_kv", "arch.head_dim",
                         "arch.n_layer", "arch.vocab",  "arch.ctx",  "arch.bos"};
  long v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int k = 0; k < 8; ++k) {
    bool found = false;
    long x = 0;
    // unreadable values count as absent here, as read_meta_i leaves them 0
    if (st.meta.count(keys[k]) && meta_int(st, path, keys[k], &x, &found) == FG_OK && found)
      v[k] = x;
  }
  for (int k = 0; k < 7; ++k)
    if (v[k] <= 0) return FG_OK;  // older checkpoint: nothing to cross-check
  const std::string canon = arch_canonical(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
  auto c = st.meta.find("arch.canonical");
  if (c != st.meta.end() && c->second != canon)
    return fail(FG_EARCH,
                "inconsistent arch metadata in %s (arch.canonical != fields): declares %s, fields "
                "give %s",
                path.c_str(), c->second.c_str(), canon.c_str());
  auto id = st.meta.find("arch.id");
  if (id != st.meta.end() && id->second != arch_id(canon))
    return fail(FG_EARCH,
                "inconsistent arch metadata in %s (arch.id != digest of fields): declares %s, "
                "fields give %s",
                path.c_str(), id->second.c_str(), arch_id(canon).c_str());
  return FG_OK;
}

// one F32 tensor of exactly `want` values into dst (st_load / st_load_into)
int32_t st_read(const StFile& st, const std::string& path, FILE* f, const std::string& name,
                size_t want, float* dst) {
  auto it = st.tensors.find(name);
  if (it == st.tensors.end())
    return fail(FG_EWEIGHT, "tensor %s in %s: not found", name.c_str(), path.c_str());
  const StEntry& e = it->second;
  if (e.dtype != "F32")
    return fail(FG_EWEIGHT, "tensor %s in %s: dtype %s, expected F32", name.c_str(), path.c_str(),
                e.dtype.c_str());
  uint64_t n = 1;
  for (uint64_t x : e.shape) n *= x;
  if (n != want || e.end < e.begin || e.end - e.begin != 4 * n)
    return fail(FG_EWEIGHT,
                "tensor %s in %s: %llu values, expected %zu (does not fit the per-layer slot: "
                "wrong arch?)",
                name.c_str(), path.c_str(), (unsigned long long)n, want);
  if (st.data0 + e.end > st.size)
    return fail(FG_EWEIGHT, "tensor %s in %s: data past the end of the file", name.c_str(),
                path.c_str());
  if (fseek(f, (long)(st.data0 + e.begin), SEEK_SET) != 0 || fread(dst, 4, want, f) != want)
    return fail(FG_EWEIGHT, "tensor %s in %s: read failed", name.c_str(), path.c_str());
  return FG_OK;
}

}  // namespace
}  // namespace fgpt

using namespace fgpt;

extern "C" int32_t fg_weights_read(const fg_dims* dims, const char* weights_dir, float* wte,
                                   float* c_q, float* c_k, float* c_v, float* c_proj, float* c_fc,
                                   float* c_proj2, float* lm_head) {
  if (!weights_dir || !wte || !c_q || !c_k || !c_v || !c_proj || !c_fc || !c_proj2 || !lm_head)
    return set_error(FG_EARG, "NULL argument");
  Dims d;
  TRY(check_dims(dims, &d));
  const std::string dir(weights_dir);
  const size_t D = d.D, qd = d.qd(), kd = d.kvd(), dff = d.dff, V = d.V, L = d.L;
  const std::string stp = dir + "/model.safetensors";
  if (file_exists(stp)) {
    StFile st;
    TRY(st_open(stp, &st));
    TRY(st_check_arch(st, stp, d));
    FILE* f = fopen(stp.c_str(), "rb");
    if (!f) return fail(FG_EWEIGHT, "cannot open %s", stp.c_str());
    int32_t rc = st_read(st, stp, f, "wte", V * D, wte);
    if (rc == FG_OK) rc = st_read(st, stp, f, "lm", V * D, lm_head);
    for (size_t l = 0; l < L && rc == FG_OK; ++l) {
      const std::string p = "l" + std::to_string(l) + ".";
      rc = st_read(st, stp, f, p + "q", qd * D, c_q + l * qd * D);
      if (rc == FG_OK) rc = st_read(st, stp, f, p + "k", kd * D, c_k + l * kd * D);
      if (rc == FG_OK) rc = st_read(st, stp, f, p + "v", kd * D, c_v + l * kd * D);
      if (rc == FG_OK) rc = st_read(st, stp, f, p + "p", D * qd, c_proj + l * D * qd);
      if (rc == FG_OK) rc = st_read(st, stp, f, p + "fc", dff * D, c_fc + l * dff * D);
      if (rc == FG_OK) rc = st_read(st, stp, f, p + "p2", D * dff, c_proj2 + l * D * dff);
    }
    fclose(f);
    return rc;
  }
  TRY(check_arch_txt(dir, d));
  TRY(read_npy_f32(dir + "/transformer_wte_weight.npy", V * D, wte));
  TRY(read_npy_f32(dir + "/lm_head_weight.npy", V * D, lm_head));
  for (size_t l = 0; l < L; ++l) {
    const std::string p = dir + "/transformer_h_" + std::to_string(l) + "_";
    TRY(read_npy_f32(p + "attn_c_q_weight.npy", qd * D, c_q + l * qd * D));
    TRY(read_npy_f32(p + "attn_c_k_weight.npy", kd * D, c_k + l * kd * D));
    TRY(read_npy_f32(p + "attn_c_v_weight.npy", kd * D, c_v + l * kd * D));
    TRY(read_npy_f32(p + "attn_c_proj_weight.npy", D * qd, c_proj + l * D * qd));
    TRY(read_npy_f32(p + "mlp_c_fc_weight.npy", dff * D, c_fc + l * dff * D));
    TRY(read_npy_f32(p + "mlp_c_proj_weight.npy", D * dff, c_proj2 + l * D * dff));
  }
  return FG_OK;
}

// eval_bpb's rows file (src/app/eval_bpb.f90:51-57,97-115): one int32 .npy
// of logical shape (N, T+1), written with fortran_order True by numpy from a
// Fortran-order array or False from a C-order one; either way row i is
// element (i, :). rows == NULL: only the shape.
extern "C" int32_t fg_rows_npy(const char* path, int32_t* n_rows, int32_t* width, int32_t* rows) {
  if (!path || !n_rows || !width) return set_error(FG_EARG, "NULL argument");
  FILE* f = fopen(path, "rb");
  if (!f) return fail(FG_EARG, "rows npy missing or empty: %s", path);
  unsigned char mg[10];
  int32_t rc = FG_OK;
  std::string hdr;
  if (fread(mg, 1, 8, f) != 8 || memcmp(mg, "\x93NUMPY", 6) != 0) {
    rc = fail(FG_EARG, "rows npy unreadable: %s", path);
  } else {
    uint32_t hlen = 0;
    if (mg[6] == 1) {
      if (fread(mg, 1, 2, f) != 2) rc = fail(FG_EARG, "rows npy unreadable: %s", path);
      hlen = mg[0] | (mg[1] << 8);
    } else {
      if (fread(mg, 1, 4, f) != 4) rc = fail(FG_EARG, "rows npy unreadable: %s", path);
      hlen = mg[0] | (mg[1] << 8) | (mg[2] << 16) | ((uint32_t)mg[3] << 24);
    }
    if (rc == FG_OK) {
      hdr.resize(hlen);
      if (hlen > 65536 || fread(&hdr[0], 1, hlen, f) != hlen)
        rc = fail(FG_EARG, "rows npy unreadable: %s", path);
    }
  }
  long long n = 0, w = 0;
  bool forder = false;
  if (rc == FG_OK) {
    const size_t p = hdr.find("'shape': (");
    if (hdr.find("'descr': '<i4'") == std::string::npos)
      rc = fail(FG_EARG, "rows npy %s: dtype is not '<i4' (int32)", path);
    else if (p == std::string::npos || sscanf(hdr.c_str() + p + 10, "%lld, %lld)", &n, &w) != 2 ||
             n < 1 || w < 2)
      rc = fail(FG_EARG, "rows npy %s: need a 2-D (N, T+1) array", path);
    else
      forder = hdr.find("'fortran_order': True") != std::string::npos;
  }
  if (rc == FG_OK && (n > INT32_MAX || w > INT32_MAX))
    rc = fail(FG_EARG, "rows npy %s: too large", path);
  if (rc == FG_OK) {
    *n_rows = (int32_t)n;
    *width = (int32_t)w;
    if (rows) {
      std::vector<int32_t> buf((size_t)(n * w));
      if (fread(buf.data(), 4, buf.size(), f) != buf.size()) {
        rc = fail(FG_EARG, "rows npy %s: truncated payload", path);
      } else if (forder) {  // column-major: element (i, j) at j*N + i
        for (long long i = 0; i < n; ++i)
          for (long long j = 0; j < w; ++j) rows[i * w + j] = buf[(size_t)(j * n + i)];
      } else {
        memcpy(rows, buf.data(), buf.size() * 4);
      }
    }
  }
  fclose(f);
  return rc;
}
