// ModelWeights::from_safetensors for the MI355X build (kernels/model_weights.cu:14-59, 80-154).
//
// Same contract as the reference: every file's tensors are mapped by name onto the
// ModelWeights fields (the name table of get_model_weights_entry, model_weights.cu:32-59),
// an unknown name is an error, a tensor may appear only once, dtype must be BF16, and after
// all files every field must be present (check_all_present, :14-30); the RoPE tables are
// built as by init_rope_buffer.  Changed on purpose:
//   * BF16 is kept (the reference converts to FP16 on the device);
//   * one 256-byte-aligned arena with the random-init layout instead of one allocation per
//     tensor, and each shape is checked against Llama-3.1-8B (the reference checks bytes only);
//   * all headers are parsed and validated before any device memory is touched, so a bad
//     checkpoint fails fast with a message (status < 0, ie_last_error) and leaves nothing
//     allocated;
//   * data is streamed with pread into two pinned staging buffers and asynchronous copies
//     (no mmap of the whole file, no pageable-memory copies).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "ie_kernels.h"

namespace ie {

namespace {

// ---------------------------------------------------------------- JSON (header subset)
// The safetensors header is a JSON object; values needed: strings, integer arrays, nested
// objects ("__metadata__").  This parser accepts any JSON value and keeps what is needed.
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  long long inum = 0;
  bool is_int = false;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const char* key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* end;
  std::string err;

  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end - p) < n || std::memcmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  bool str(std::string& out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    out.clear();
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) return fail("bad escape");
        switch (*p) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {  // kept as-is: tensor names are ASCII
            if (end - p < 5) return fail("bad \\u escape");
            out.append(p - 1, 6);
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
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 16) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    if (*p == '{') {
      v.kind = JVal::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      while (true) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        v.obj.emplace_back(std::move(k), JVal{});
        if (!value(v.obj.back().second, depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      v.kind = JVal::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      while (true) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') {
      v.kind = JVal::Str;
      return str(v.str);
    }
    if (lit("true")) {
      v.kind = JVal::Bool;
      v.num = 1;
      return true;
    }
    if (lit("false")) {
      v.kind = JVal::Bool;
      return true;
    }
    if (lit("null")) return true;
    // number
    const char* s = p;
    if (p < end && (*p == '-' || *p == '+')) ++p;
    bool frac = false;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                       *p == '-' || *p == '+')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      ++p;
    }
    if (p == s) return fail("unexpected character");
    const std::string t(s, p);
    v.kind = JVal::Num;
    v.num = std::strtod(t.c_str(), nullptr);
    if (!frac) {
      v.is_int = true;
      v.inum = std::strtoll(t.c_str(), nullptr, 10);
    }
    return true;
  }
};

// ---------------------------------------------------------------- tensor name table
struct Target {
  ie_bf16** slot;
  std::vector<long long> shape;
  std::string name;
};

// model_weights.cu:32-59: HF Llama tensor names -> ModelWeights fields (plus the expected
// Llama-3.1-8B shape of each).
bool target_of(ie_model_weights& m, const std::string& name, Target& t, std::string& err) {
  const long long H = kHidden, F = kFFN, V = kVocab, KV = kKVDim;
  t.name = name;
  if (name == "model.embed_tokens.weight") {
    t.slot = &m.emb_lookup;
    t.shape = {V, H};
    return true;
  }
  if (name == "model.norm.weight") {
    t.slot = &m.final_norm;
    t.shape = {H};
    return true;
  }
  if (name == "lm_head.weight") {
    t.slot = &m.lm_head;
    t.shape = {V, H};
    return true;
  }
  const std::string pre = "model.layers.";
  if (name.compare(0, pre.size(), pre) == 0) {
    const size_t dot = name.find('.', pre.size());
    const std::string num = name.substr(pre.size(), dot == std::string::npos ? std::string::npos
                                                                              : dot - pre.size());
    bool digits = !num.empty() && num.size() <= 3;
    for (char c : num) digits = digits && c >= '0' && c <= '9';
    if (dot != std::string::npos && digits) {
      const int layer = std::stoi(num);
      if (layer < 0 || layer >= kLayers) {
        err = name + ": layer index out of range [0, 32)";
        return false;
      }
      static const struct {
        const char* sub;
        int field;
      } subs[] = {{"input_layernorm.weight", 0},       {"self_attn.q_proj.weight", 1},
                  {"self_attn.k_proj.weight", 2},      {"self_attn.v_proj.weight", 3},
                  {"self_attn.o_proj.weight", 4},      {"post_attention_layernorm.weight", 5},
                  {"mlp.gate_proj.weight", 6},         {"mlp.up_proj.weight", 7},
                  {"mlp.down_proj.weight", 8}};
      const std::string sub = name.substr(dot + 1);
      for (const auto& s : subs) {
        if (sub == s.sub) {
          t.slot = layer_field(m.layers[layer], s.field);
          const long long shapes[kLayerFields][2] = {{H, 0}, {H, H}, {KV, H}, {KV, H}, {H, H},
                                                     {H, 0}, {F, H}, {F, H}, {H, F}};
          t.shape = {shapes[s.field][0]};
          if (shapes[s.field][1]) t.shape.push_back(shapes[s.field][1]);
          return true;
        }
      }
    }
  }
  err = name + " is an unknown tensor name";  // model_weights.cu:58
  return false;
}

std::string shape_str(const std::vector<long long>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

struct Entry {
  int file;
  ie_bf16** slot;  // in the staging ModelWeights (offsets into the arena once assigned)
  size_t file_offset;
  size_t bytes;
  std::string name;
};

struct FileCloser {
  std::vector<int> fds;
  ~FileCloser() {
    for (int fd : fds)
      if (fd >= 0) close(fd);
  }
};

bool read_full(int fd, void* dst, size_t n, size_t off) {
  char* d = static_cast<char*>(dst);
  while (n) {
    const ssize_t r = pread(fd, d, n, (off_t)off);
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
    off += (size_t)r;
  }
  return true;
}

}  // namespace

int load_safetensors(ie_model_weights* out, const char* const* paths, int n_paths) {
  IE_REQUIRE(out != nullptr, "from_safetensors: null output");
  IE_REQUIRE(paths != nullptr && n_paths >= 1, "from_safetensors: no files");
  std::memset(out, 0, sizeof *out);

  // ---- pass 1: every header, validated against the name table, before any device work
  ie_model_weights m{};  // fields hold 1-based "present" marks during validation
  std::vector<Entry> entries;
  FileCloser files;
  for (int fi = 0; fi < n_paths; ++fi) {
    IE_REQUIRE(paths[fi] != nullptr, "from_safetensors: path %d is null", fi);
    const int fd = open(paths[fi], O_RDONLY);
    files.fds.push_back(fd);
    IE_REQUIRE(fd >= 0, "from_safetensors: cannot open %s", paths[fi]);
    struct stat st {};
    IE_REQUIRE(fstat(fd, &st) == 0, "from_safetensors: cannot stat %s", paths[fi]);
    const size_t fsize = (size_t)st.st_size;
    uint64_t hlen = 0;
    IE_REQUIRE(fsize >= 8 && read_full(fd, &hlen, 8, 0),
               "from_safetensors: %s: too short for a header", paths[fi]);
    IE_REQUIRE(hlen >= 2 && hlen <= (100ull << 20) && 8 + hlen <= fsize,
               "from_safetensors: %s: header length %llu out of range", paths[fi],
               (unsigned long long)hlen);
    std::string hdr(hlen, '\0');
    IE_REQUIRE(read_full(fd, hdr.data(), hlen, 8), "from_safetensors: %s: header read failed",
               paths[fi]);
    JVal root;
    JParser jp{hdr.data(), hdr.data() + hdr.size(), {}};
    IE_REQUIRE(jp.value(root, 0) && root.kind == JVal::Obj,
               "from_safetensors: %s: bad header JSON (%s)", paths[fi],
               jp.err.empty() ? "not an object" : jp.err.c_str());
    const size_t data0 = 8 + hlen;
    for (const auto& kv : root.obj) {
      if (kv.first == "__metadata__") continue;
      Target t{};
      std::string err;
      IE_REQUIRE(target_of(m, kv.first, t, err), "from_safetensors: %s: %s", paths[fi],
                 err.c_str());
      IE_REQUIRE(*t.slot == nullptr, "from_safetensors: %s: tensor %s appears twice", paths[fi],
                 kv.first.c_str());
      const JVal& v = kv.second;
      const JVal* dt = v.get("dtype");
      const JVal* sh = v.get("shape");
      const JVal* off = v.get("data_offsets");
      IE_REQUIRE(v.kind == JVal::Obj && dt && dt->kind == JVal::Str && sh &&
                     sh->kind == JVal::Arr && off && off->kind == JVal::Arr && off->arr.size() == 2,
                 "from_safetensors: %s: tensor %s: malformed entry", paths[fi], kv.first.c_str());
      IE_REQUIRE(dt->str == "BF16", "from_safetensors: %s: tensor %s has dtype %s, expected BF16",
                 paths[fi], kv.first.c_str(), dt->str.c_str());  // model_weights.cu:118
      std::vector<long long> shape;
      for (const JVal& d : sh->arr) {
        IE_REQUIRE(d.kind == JVal::Num && d.is_int && d.inum >= 0,
                   "from_safetensors: %s: tensor %s: bad shape", paths[fi], kv.first.c_str());
        shape.push_back(d.inum);
      }
      IE_REQUIRE(shape == t.shape, "from_safetensors: %s: tensor %s has shape %s, expected %s",
                 paths[fi], kv.first.c_str(), shape_str(shape).c_str(),
                 shape_str(t.shape).c_str());
      size_t numel = 1;
      for (long long d : shape) numel *= (size_t)d;
      const JVal &o0 = off->arr[0], &o1 = off->arr[1];
      IE_REQUIRE(o0.kind == JVal::Num && o0.is_int && o1.kind == JVal::Num && o1.is_int &&
                     o0.inum >= 0 && o1.inum >= o0.inum,
                 "from_safetensors: %s: tensor %s: bad data_offsets", paths[fi], kv.first.c_str());
      const size_t b0 = (size_t)o0.inum, b1 = (size_t)o1.inum;
      IE_REQUIRE(b1 - b0 == numel * 2,  // model_weights.cu:124-126
                 "from_safetensors: %s: tensor %s: %zu data bytes for %zu bf16 elements", paths[fi],
                 kv.first.c_str(), b1 - b0, numel);
      IE_REQUIRE(data0 + b1 <= fsize, "from_safetensors: %s: tensor %s runs past the end of the file",
                 paths[fi], kv.first.c_str());
      *t.slot = reinterpret_cast<ie_bf16*>(entries.size() + 1);  // mark present
      entries.push_back({fi, t.slot, data0 + b0, numel * 2, kv.first});
    }
  }
  // check_all_present (model_weights.cu:14-30), naming the first missing tensor
  {
    auto missing = [&](ie_bf16* p, const std::string& n) {
      if (!p) set_error("from_safetensors: missing tensor %s", n.c_str());
      return !p;
    };
    if (missing(m.emb_lookup, "model.embed_tokens.weight") ||
        missing(m.final_norm, "model.norm.weight") || missing(m.lm_head, "lm_head.weight"))
      return IE_ERR_INVALID_ARG;
    static const char* subs[kLayerFields] = {
        "input_layernorm.weight", "self_attn.q_proj.weight",     "self_attn.k_proj.weight",
        "self_attn.v_proj.weight", "self_attn.o_proj.weight",    "post_attention_layernorm.weight",
        "mlp.gate_proj.weight",    "mlp.up_proj.weight",         "mlp.down_proj.weight"};
    for (int l = 0; l < kLayers; ++l)
      for (int f = 0; f < kLayerFields; ++f)
        if (missing(*layer_field(m.layers[l], f),
                    "model.layers." + std::to_string(l) + "." + subs[f]))
          return IE_ERR_INVALID_ARG;
  }

  // ---- pass 2: arena, then stream every tensor through pinned staging buffers
  void* arena = nullptr;
  IE_CHECK_HIP(hipMalloc(&arena, weights_arena_bytes()));
  ie_model_weights w{};
  weights_arena_assign(&w, arena);
  // the staging ModelWeights `m` and the arena-backed `w` have the same field layout: the
  // destination of an entry is the field at the same offset within the struct
  auto dest_of = [&](ie_bf16** slot_in_m) {
    const size_t off = (size_t)(reinterpret_cast<char*>(slot_in_m) - reinterpret_cast<char*>(&m));
    return *reinterpret_cast<ie_bf16**>(reinterpret_cast<char*>(&w) + off);
  };
  constexpr size_t kChunk = 64ull << 20;
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  hipStream_t st = nullptr;
  int rc = IE_OK;
  auto fail = [&](int code, const char* fmt, const char* a, const char* b) {
    set_error(fmt, a, b);
    rc = code;
  };
  if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess ||
      hipHostMalloc(&stage[0], kChunk, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc(&stage[1], kChunk, hipHostMallocDefault) != hipSuccess ||
      hipEventCreateWithFlags(&done[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&done[1], hipEventDisableTiming) != hipSuccess)
    fail(IE_ERR_HIP, "from_safetensors: %s%s", "staging setup failed", "");
  int buf = 0;
  bool used[2] = {false, false};
  for (size_t e = 0; e < entries.size() && rc == IE_OK; ++e) {
    const Entry& en = entries[e];
    char* dst = reinterpret_cast<char*>(dest_of(en.slot));
    for (size_t done_b = 0; done_b < en.bytes && rc == IE_OK;) {
      const size_t n = std::min(kChunk, en.bytes - done_b);
      if (used[buf] && hipEventSynchronize(done[buf]) != hipSuccess) {
        fail(IE_ERR_HIP, "from_safetensors: %s%s", "copy failed", "");
        break;
      }
      if (!read_full(files.fds[en.file], stage[buf], n, en.file_offset + done_b)) {
        fail(IE_ERR_INVALID_ARG, "from_safetensors: read of %s failed (%s)", en.name.c_str(),
             paths[en.file]);
        break;
      }
      if (hipMemcpyAsync(dst + done_b, stage[buf], n, hipMemcpyHostToDevice, st) != hipSuccess ||
          hipEventRecord(done[buf], st) != hipSuccess) {
        fail(IE_ERR_HIP, "from_safetensors: %s%s", "copy failed", "");
        break;
      }
      used[buf] = true;
      buf ^= 1;
      done_b += n;
    }
  }
  if (st && hipStreamSynchronize(st) != hipSuccess && rc == IE_OK)
    fail(IE_ERR_HIP, "from_safetensors: %s%s", "copy failed", "");
  for (int i = 0; i < 2; ++i) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  if (st) (void)hipStreamDestroy(st);
  if (rc == IE_OK) rc = weights_upload_rope(&w);  // init_rope_buffer (model_weights.cu:147)
  if (rc != IE_OK) {
    (void)hipFree(arena);
    return rc;
  }
  *out = w;
  return IE_OK;
}

}  // namespace ie
