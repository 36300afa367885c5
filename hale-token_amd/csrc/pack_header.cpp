// pack_header.cpp -- the Hale expert pack header (src/expert/pack.rs:55-123):
// the JSON PackHeader reader and record offsets.  Host-only C++ with no HIP
// dependency, so the parser also builds on its own (the sanitizer test).
#include "pack_header.h"

#include <stdint.h>

#include "../../include/hale_moe.h"

namespace hale {

namespace {

// A small JSON reader for the header: objects, arrays, strings, unsigned
// integers, and (skipped) other literals.
struct Json {
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool expect(char c) {
    ws();
    if (p < end && *p == c) {
      p++;
      return true;
    }
    err = std::string("expected '") + c + "'";
    return false;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  bool string(std::string* out) {
    if (!expect('"')) return false;
    out->clear();
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) break;
        switch (*p) {
          case 'n': out->push_back('\n'); break;
          case 't': out->push_back('\t'); break;
          case 'r': out->push_back('\r'); break;
          case 'b': out->push_back('\b'); break;
          case 'f': out->push_back('\f'); break;
          case 'u':  // kept verbatim: no header field needs it
            out->append("\\u");
            break;
          default: out->push_back(*p);
        }
        p++;
      } else {
        out->push_back(*p++);
      }
    }
    if (p >= end) {
      err = "unterminated string";
      return false;
    }
    p++;
    return true;
  }
  bool uint(size_t* out) {
    ws();
    if (p >= end || *p < '0' || *p > '9') {
      err = "expected an unsigned integer";
      return false;
    }
    size_t v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const size_t d = (size_t)(*p - '0');
      if (v > (SIZE_MAX - d) / 10) {
        err = "integer out of range";
        return false;
      }
      v = v * 10 + d;
      p++;
    }
    if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
      err = "expected an integer";
      return false;
    }
    *out = v;
    return true;
  }
  // skips any value
  bool skip(int depth = 0) {
    if (depth > 64) {
      err = "nesting too deep";
      return false;
    }
    ws();
    if (p >= end) {
      err = "unexpected end";
      return false;
    }
    if (*p == '"') {
      std::string s;
      return string(&s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      p++;
      if (peek(close)) {
        p++;
        return true;
      }
      for (;;) {
        if (obj) {
          std::string k;
          if (!string(&k) || !expect(':')) return false;
        }
        if (!skip(depth + 1)) return false;
        if (peek(',')) {
          p++;
          continue;
        }
        return expect(close);
      }
    }
    const char* start = p;
    while (p < end && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\t' &&
           *p != '\n' && *p != '\r')
      p++;
    if (p == start) {
      err = "expected a value";
      return false;
    }
    return true;
  }
};

int dtype_of(const std::string& s) {
  // DType's serde names (src/tensor/dtype.rs:13-25)
  if (s == "f32") return HALE_F32;
  if (s == "f16") return HALE_F16;
  if (s == "bf16") return HALE_BF16;
  if (s == "q8_0") return HALE_Q8_0;
  if (s == "q4_0") return HALE_Q4_0;
  return -1;
}

}  // namespace

bool PackHeader::file_size_checked(size_t* out) const {
  size_t n = 0;
  return !__builtin_mul_overflow(moe_layers.size(), num_experts, &n) &&
         !__builtin_mul_overflow(n, record_stride, &n) && !__builtin_add_overflow(n, data_offset, out);
}

bool parse_pack_header(const char* json, size_t len, PackHeader* h, std::string* err) {
  Json j{json, json + len, {}};
  enum { VERSION, DTYPE, HIDDEN, INTER, EXPERTS, LAYERS, RBYTES, RSTRIDE, DOFF, NF };
  bool seen[NF] = {};
  auto fail = [&](const std::string& m) {
    *err = m;
    return false;
  };
  if (!j.expect('{')) return fail(j.err);
  if (!j.peek('}')) {
    for (;;) {
      std::string key;
      if (!j.string(&key) || !j.expect(':')) return fail(j.err);
      size_t v = 0;
      bool ok = true;
      if (key == "version") {
        ok = j.uint(&v);
        if (ok && v > UINT32_MAX) return fail("version out of range");
        h->version = (uint32_t)v;
        seen[VERSION] = true;
      } else if (key == "dtype") {
        std::string s;
        ok = j.string(&s);
        if (ok && (h->dtype = dtype_of(s)) < 0) return fail("unknown dtype \"" + s + "\"");
        seen[DTYPE] = true;
      } else if (key == "hidden_size") {
        ok = j.uint(&h->hidden);
        seen[HIDDEN] = true;
      } else if (key == "intermediate_size") {
        ok = j.uint(&h->inter);
        seen[INTER] = true;
      } else if (key == "num_experts") {
        ok = j.uint(&h->num_experts);
        seen[EXPERTS] = true;
      } else if (key == "moe_layers") {
        h->moe_layers.clear();
        ok = j.expect('[');
        if (ok && j.peek(']')) {
          j.p++;
        } else {
          while (ok) {
            ok = j.uint(&v);
            if (!ok) break;
            h->moe_layers.push_back(v);
            if (j.peek(',')) {
              j.p++;
              continue;
            }
            ok = j.expect(']');
            break;
          }
        }
        seen[LAYERS] = true;
      } else if (key == "record_bytes") {
        ok = j.uint(&h->record_bytes);
        seen[RBYTES] = true;
      } else if (key == "record_stride") {
        ok = j.uint(&h->record_stride);
        seen[RSTRIDE] = true;
      } else if (key == "data_offset") {
        ok = j.uint(&h->data_offset);
        seen[DOFF] = true;
      } else {
        ok = j.skip();  // unknown fields are ignored, as serde does by default
      }
      if (!ok) return fail(key + ": " + j.err);
      if (j.peek(',')) {
        j.p++;
        continue;
      }
      if (!j.expect('}')) return fail(j.err);
      break;
    }
  } else {
    j.p++;
  }
  static const char* names[NF] = {"version", "dtype", "hidden_size", "intermediate_size",
                                  "num_experts", "moe_layers", "record_bytes", "record_stride",
                                  "data_offset"};
  for (int i = 0; i < NF; i++)
    if (!seen[i]) return fail(std::string("missing field `") + names[i] + "`");
  j.ws();
  if (j.p != j.end) return fail("trailing characters after the header");
  size_t fs;
  if (!h->file_size_checked(&fs)) return fail("header sizes overflow the file size");
  return true;
}

bool pack_offset_of(const PackHeader& h, uint32_t layer, uint32_t expert, uint64_t* off,
                    std::string* err) {
  size_t ordinal = h.moe_layers.size();
  for (size_t i = 0; i < h.moe_layers.size(); i++)
    if (h.moe_layers[i] == layer) {
      ordinal = i;
      break;
    }
  if (ordinal == h.moe_layers.size()) {
    *err = "layer " + std::to_string(layer) + " has no experts in the pack";
    return false;
  }
  if (expert >= h.num_experts) {
    *err = "expert L" + std::to_string(layer) + "E" + std::to_string(expert) + " out of range";
    return false;
  }
  const size_t index = ordinal * h.num_experts + expert;
  *off = (uint64_t)(h.data_offset + index * h.record_stride);
  return true;
}

}  // namespace hale
