// checkpoint.cpp -- safetensors reader and weight loader of the C++ mirror
// (mi_bridge::SafetensorsFile, mi_bridge::load_weights).
//
// Reference: cpp/src/Checkpoint.cpp.  The file format is safetensors: an 8-byte
// little-endian header length, a JSON header mapping tensor names to
// {dtype, shape, data_offsets}, then the payload (Checkpoint.cpp:229-299,331-400).
// Two layouts are read (Checkpoint.cpp:404-570):
//   * a Python/MLX file (it holds "tok_embeddings.weight"): nn.Linear [out, in]
//     matrices, fused attention.wqkv [q + 2 kv, H] and feed_forward.w12 [2 I, H];
//     each engine matrix [in, out] is a row range of a file matrix, transposed;
//   * an engine file: the engine's own names and [in, out] layout (get_model_tensors,
//     Checkpoint.cpp:147-174), copied with a dtype conversion only.
// The file is memory-mapped; each tensor's bytes are copied once to a device staging
// buffer and mi_convert_matrix does the row slice, transpose and dtype conversion on
// the GPU into the caller's buffers (the reference transposes on the CPU).
//
// The header is parsed as JSON (objects, arrays, strings with escapes, numbers,
// literals) rather than by searching for key strings, so a tensor name that is a
// prefix or a substring of another cannot pick up the wrong entry.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/gemm_bridge.hpp"
#include "../../include/mi_gemm.h"

namespace mi_bridge {

namespace {

// ---- minimal JSON reader for the header ---------------------------------------

struct JsonCursor {
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool expect(char c) {
    ws();
    if (p < end && *p == c) {
      ++p;
      return true;
    }
    if (err.empty()) err = std::string("expected '") + c + "'";
    return false;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  static void put_utf8(std::string& s, unsigned cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(unsigned& v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& out) {
    if (!expect('"')) return false;
    out.clear();
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) break;
        const char e = *p++;
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
            unsigned cp = 0;
            if (!hex4(cp)) return err = "bad \\u escape", false;
            if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
              unsigned lo = 0;
              if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return err = "lone surrogate", false;
              p += 2;
              if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return err = "bad surrogate", false;
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            }
            put_utf8(out, cp);
            break;
          }
          default: return err = "bad escape", false;
        }
      } else {
        out += *p++;
      }
    }
    if (p >= end) return err = "unterminated string", false;
    ++p;
    return true;
  }
  // Non-negative integer (all the header's numbers: shapes and byte offsets).
  bool uint(uint64_t& v) {
    ws();
    if (p >= end || *p < '0' || *p > '9') return err = "expected a non-negative integer", false;
    v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = (uint64_t)(*p++ - '0');
      if (v > (UINT64_MAX - d) / 10) return err = "integer overflow", false;
      v = v * 10 + d;
    }
    return true;
  }
  // Skips any JSON value (metadata entries, unknown keys).
  bool skip(int depth = 0) {
    if (depth > 64) return err = "nesting too deep", false;
    ws();
    if (p >= end) return err = "unexpected end", false;
    if (*p == '"') {
      std::string s;
      return string(s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      ++p;
      if (peek(close)) return ++p, true;
      for (;;) {
        if (obj) {
          std::string k;
          if (!string(k) || !expect(':')) return false;
        }
        if (!skip(depth + 1)) return false;
        if (peek(',')) {
          ++p;
          continue;
        }
        return expect(close);
      }
    }
    // number or literal
    const char* s = p;
    while (p < end && (std::strchr("+-.0123456789eE", *p) || (*p >= 'a' && *p <= 'z'))) ++p;
    if (p == s) return err = "bad value", false;
    return true;
  }
};

bool parse_header(const char* text, size_t len, std::vector<TensorInfo>& out, std::string& err) {
  JsonCursor c{text, text + len, {}};
  out.clear();
  if (!c.expect('{')) return err = c.err, false;
  if (c.peek('}')) return true;
  for (;;) {
    std::string name;
    if (!c.string(name) || !c.expect(':')) return err = c.err, false;
    if (name == "__metadata__") {
      if (!c.skip()) return err = c.err, false;
    } else {
      TensorInfo t;
      t.name = name;
      bool have_dtype = false, have_shape = false, have_offsets = false;
      if (!c.expect('{')) return err = c.err + " in '" + name + "'", false;
      if (!c.peek('}')) {
        for (;;) {
          std::string key;
          if (!c.string(key) || !c.expect(':')) return err = c.err, false;
          if (key == "dtype") {
            if (!c.string(t.dtype)) return err = c.err, false;
            have_dtype = true;
          } else if (key == "shape" || key == "data_offsets") {
            std::vector<uint64_t> vals;
            if (!c.expect('[')) return err = c.err, false;
            if (!c.peek(']')) {
              for (;;) {
                uint64_t v = 0;
                if (!c.uint(v)) return err = c.err + " in '" + name + "'", false;
                vals.push_back(v);
                if (c.peek(',')) {
                  ++c.p;
                  continue;
                }
                break;
              }
            }
            if (!c.expect(']')) return err = c.err, false;
            if (key == "shape") {
              t.shape.assign(vals.begin(), vals.end());
              have_shape = true;
            } else {
              if (vals.size() != 2) return err = "data_offsets of '" + name + "' must hold 2 values", false;
              t.begin = (size_t)vals[0];
              t.end = (size_t)vals[1];
              have_offsets = true;
            }
          } else if (!c.skip()) {
            return err = c.err, false;
          }
          if (c.peek(',')) {
            ++c.p;
            continue;
          }
          break;
        }
      }
      if (!c.expect('}')) return err = c.err, false;
      if (!have_dtype || !have_shape || !have_offsets)
        return err = "tensor '" + name + "' lacks dtype, shape or data_offsets", false;
      out.push_back(std::move(t));
    }
    if (c.peek(',')) {
      ++c.p;
      continue;
    }
    break;
  }
  if (!c.expect('}')) return err = c.err, false;
  c.ws();
  if (c.p != c.end) return err = "trailing bytes after the header object", false;
  return true;
}

size_t dtype_bytes(const std::string& d) {
  if (d == "F32") return 4;
  if (d == "BF16" || d == "F16") return 2;
  return 0;
}

int dtype_code(const std::string& d) { return d == "BF16" ? MI_BF16 : d == "F16" ? MI_F16 : MI_F32; }

// Device staging buffer for one tensor's file bytes, per thread, grown on demand.
thread_local void* t_stage = nullptr;
thread_local size_t t_stage_bytes = 0;

bool stage(size_t bytes) {
  if (bytes <= t_stage_bytes) return true;
  if (t_stage) (void)hipFree(t_stage);
  t_stage = nullptr;
  t_stage_bytes = 0;
  if (hipMalloc(&t_stage, bytes) != hipSuccess) return false;
  t_stage_bytes = bytes;
  return true;
}

}  // namespace

// ---- SafetensorsFile -------------------------------------------------------------

SafetensorsFile::~SafetensorsFile() { close(); }

void SafetensorsFile::close() {
  if (map_) munmap(map_, size_);
  map_ = nullptr;
  size_ = 0;
  payload_ = 0;
  tensors_.clear();
}

bool SafetensorsFile::open(const std::string& path) {
  close();
  err_.clear();
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return err_ = "cannot open " + path, false;
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    return err_ = path + " is not a safetensors file (shorter than 8 bytes)", false;
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return err_ = "cannot map " + path, false;
  map_ = (uint8_t*)m;
  size_ = (size_t)st.st_size;
  uint64_t hlen = 0;
  std::memcpy(&hlen, map_, 8);  // little-endian, as the format and this host are
  // The reference caps the header at 10 MiB (Checkpoint.cpp:394-396); so does this reader.
  if (hlen == 0 || hlen > (10u << 20) || hlen > size_ - 8) {
    close();
    return err_ = "bad header length in " + path, false;
  }
  payload_ = 8 + (size_t)hlen;
  std::string perr;
  if (!parse_header((const char*)map_ + 8, (size_t)hlen, tensors_, perr)) {
    close();
    return err_ = "header of " + path + ": " + perr, false;
  }
  for (const TensorInfo& t : tensors_) {
    size_t n = 1;
    bool overflow = false;
    for (size_t d : t.shape) overflow = overflow || __builtin_mul_overflow(n, d, &n);
    const size_t es = dtype_bytes(t.dtype);
    if (overflow || t.end < t.begin || t.end > size_ - payload_ ||
        (es && t.end - t.begin != n * es)) {
      const std::string name = t.name;
      close();
      return err_ = "tensor '" + name + "' has offsets outside the payload or a size that does "
                    "not match its shape",
             false;
    }
  }
  return true;
}

const TensorInfo* SafetensorsFile::find(const std::string& name) const {
  for (const TensorInfo& t : tensors_)
    if (t.name == name) return &t;
  return nullptr;
}

const uint8_t* SafetensorsFile::data(const TensorInfo& t) const { return map_ + payload_ + t.begin; }

bool SafetensorsFile::is_python_format() const { return find("tok_embeddings.weight") != nullptr; }

// ---- load_weights ------------------------------------------------------------------

namespace {

struct Loader {
  const SafetensorsFile& f;
  int dst_dtype;
  hipStream_t st;
  std::string err;

  struct Range {
    size_t row0, rows;
    void* dst;
  };

  // Copies rows [row0, row0 + rows) of the file matrix `name` (expected shape
  // file_rows x cols, or a vector when file_rows == 0) into dst, transposed or not.
  bool put(const std::string& name, size_t file_rows, size_t cols, size_t row0, size_t rows,
           bool transpose, void* dst, bool required = true) {
    return put_ranges(name, file_rows, cols, {{row0, rows, dst}}, transpose, required);
  }

  // Several row ranges of one file matrix (the de-fused rows of wqkv or w12): the
  // tensor is staged once and the ranges go out in one mi_convert_matrices call.
  bool put_ranges(const std::string& name, size_t file_rows, size_t cols, const std::vector<Range>& ranges,
                  bool transpose, bool required = true) {
    const TensorInfo* t = f.find(name);
    if (!t) {
      if (!required) return true;
      return err = "tensor '" + name + "' not found", false;
    }
    const bool vec = file_rows == 0;
    const std::vector<size_t> want = vec ? std::vector<size_t>{cols} : std::vector<size_t>{file_rows, cols};
    if (t->shape != want) {
      std::string got;
      for (size_t d : t->shape) got += std::to_string(d) + " ";
      return err = "tensor '" + name + "' has shape [ " + got + "]", false;
    }
    if (!dtype_bytes(t->dtype)) return err = "tensor '" + name + "' has dtype " + t->dtype, false;
    for (const Range& r : ranges)
      if (!r.dst) return err = "no destination for '" + name + "'", false;
    const size_t bytes = t->end - t->begin;
    // The staging buffer is reused (and freed when it grows): the previous
    // conversion, which reads it on `st`, must be done first.
    if (hipStreamSynchronize(st) != hipSuccess) return err = "stream error before '" + name + "'", false;
    if (!stage(bytes)) return err = "cannot allocate the staging buffer", false;
    if (hipMemcpy(t_stage, f.data(*t), bytes, hipMemcpyHostToDevice) != hipSuccess)
      return err = "copy of '" + name + "' to the device failed", false;
    std::vector<mi_convert_job> jobs;
    for (const Range& r : ranges) {
      const int64_t R = vec ? 1 : (int64_t)r.rows, C = (int64_t)cols;
      mi_convert_job j{};
      j.src = t_stage;
      j.src_dtype = dtype_code(t->dtype);
      j.transpose = transpose ? 1 : 0;
      j.src_ld = C;
      j.row0 = vec ? 0 : (int64_t)r.row0;
      j.rows = R;
      j.cols = C;
      j.dst = r.dst;
      j.dst_dtype = dst_dtype;
      j.dst_ld = transpose ? R : C;
      jobs.push_back(j);
    }
    const int s = mi_convert_matrices(st, jobs.data(), (int64_t)jobs.size());
    if (s != MI_OK) return err = "converting '" + name + "': " + mi_last_error(), false;
    return true;
  }
};

}  // namespace

bool load_weights(const std::string& path, const ModelConfig& c, const ModelWeights& w) {
  SafetensorsFile f;
  if (!f.open(path)) {
    std::fprintf(stderr, "[mi_bridge] load_weights: %s\n", f.error().c_str());
    return false;
  }
  if (w.layers.size() != c.n_layers) {
    std::fprintf(stderr, "[mi_bridge] load_weights: %zu layer buffers for %zu layers\n",
                 w.layers.size(), c.n_layers);
    return false;
  }
  Loader L{f, w.dtype == DType::BF16 ? MI_BF16 : MI_F32, (hipStream_t)stream(), {}};
  const size_t H = c.hidden_dim, V = c.vocab_size, I = c.intermediate_dim;
  const size_t q = c.n_heads * c.head_dim, kv = c.n_kv_heads * c.head_dim;
  bool ok = true;
  if (f.is_python_format()) {  // Checkpoint.cpp:532-570
    ok = ok && L.put("tok_embeddings.weight", V, H, 0, V, false, w.token_embeddings);
    ok = ok && L.put("output.weight", V, H, 0, V, true, w.output_projection);
    ok = ok && L.put("norm.weight", 0, H, 0, 1, false, w.final_norm);
    for (size_t l = 0; ok && l < c.n_layers; ++l) {
      const std::string p = "layers." + std::to_string(l) + ".";
      const LayerWeights& lw = w.layers[l];
      ok = ok && L.put(p + "attention_norm.weight", 0, H, 0, 1, false, lw.attn_norm);
      ok = ok && L.put(p + "ffn_norm.weight", 0, H, 0, 1, false, lw.ffn_norm);
      ok = ok && L.put(p + "attention.wo.weight", H, q, 0, H, true, lw.Wo);
      ok = ok && L.put(p + "feed_forward.w3.weight", H, I, 0, H, true, lw.w_down);
      // de-fused wqkv rows: Wq [0, q), Wk [q, q + kv), Wv [q + kv, q + 2 kv)
      ok = ok && L.put_ranges(p + "attention.wqkv.weight", q + 2 * kv, H,
                              {{0, q, lw.Wq}, {q, kv, lw.Wk}, {q + kv, kv, lw.Wv}}, true);
      // de-fused w12 rows: w_gate [0, I), w_up [I, 2 I)
      ok = ok && L.put_ranges(p + "feed_forward.w12.weight", 2 * I, H, {{0, I, lw.w_gate}, {I, I, lw.w_up}}, true);
    }
  } else {  // engine names and layout (Checkpoint.cpp:147-174, 331-388)
    ok = ok && L.put("token_embeddings", V, H, 0, V, false, w.token_embeddings);
    ok = ok && L.put("output_projection", H, V, 0, H, false, w.output_projection);
    ok = ok && L.put("final_norm.weight", 0, H, 0, 1, false, w.final_norm);
    for (size_t l = 0; ok && l < c.n_layers; ++l) {
      const std::string p = "layers." + std::to_string(l) + ".";
      const LayerWeights& lw = w.layers[l];
      ok = ok && L.put(p + "attn_norm.weight", 0, H, 0, 1, false, lw.attn_norm);
      ok = ok && L.put(p + "attn.Wq", H, q, 0, H, false, lw.Wq);
      ok = ok && L.put(p + "attn.Wk", H, kv, 0, H, false, lw.Wk);
      ok = ok && L.put(p + "attn.Wv", H, kv, 0, H, false, lw.Wv);
      ok = ok && L.put(p + "attn.Wo", q, H, 0, q, false, lw.Wo);
      ok = ok && L.put(p + "ffn_norm.weight", 0, H, 0, 1, false, lw.ffn_norm);
      ok = ok && L.put(p + "w_gate", H, I, 0, H, false, lw.w_gate);
      ok = ok && L.put(p + "w_up", H, I, 0, H, false, lw.w_up);
      ok = ok && L.put(p + "w_down", I, H, 0, I, false, lw.w_down);
    }
  }
  if (ok && hipStreamSynchronize(L.st) != hipSuccess) {
    L.err = "device error while converting";
    ok = false;
  }
  if (!ok) std::fprintf(stderr, "[mi_bridge] load_weights: %s (%s)\n", L.err.c_str(), path.c_str());
  return ok;
}

}  // namespace mi_bridge
