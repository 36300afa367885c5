// Runs the pack header reader (hale-token_amd/csrc/pack_header.cpp) over
// malformed, truncated and mutated headers.  Built with AddressSanitizer
// and UndefinedBehaviorSanitizer by tests/test_sanitizers.py, so an
// out-of-bounds read, an overflow or undefined behaviour ends the run with
// a report.  Every input lives in a heap block of exactly its length, so a
// read one byte past the header is caught.  Prints "<accepted> <rejected>";
// exits 1 if a fixed case is classified wrongly.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "pack_header.h"

namespace {

const std::string VALID =
    "{\"version\":1,\"dtype\":\"q4_0\",\"hidden_size\":64,\"intermediate_size\":32,"
    "\"num_experts\":3,\"moe_layers\":[0,1],\"record_bytes\":3456,\"record_stride\":16384,"
    "\"data_offset\":16384}";

uint64_t rng_state = 0x9E3779B97F4A7C15ull;
uint64_t next() {  // xorshift64*
  rng_state ^= rng_state >> 12;
  rng_state ^= rng_state << 25;
  rng_state ^= rng_state >> 27;
  return rng_state * 0x2545F4914F6CDD1Dull;
}

long accepted = 0, rejected = 0;

bool parse(const std::string& s) {
  char* buf = (char*)malloc(s.size() ? s.size() : 1);
  memcpy(buf, s.data(), s.size());
  hale::PackHeader h;
  std::string err;
  const bool ok = hale::parse_pack_header(buf, s.size(), &h, &err);
  free(buf);
  if (ok) {
    accepted++;
    size_t fs = 0;
    if (!h.file_size_checked(&fs) || fs != h.file_size()) {
      fprintf(stderr, "accepted a header whose file size overflows\n");
      exit(1);
    }
    for (uint32_t l = 0; l < 4; l++)
      for (uint32_t e = 0; e < 4; e++) {
        uint64_t off = 0;
        if (hale::pack_offset_of(h, l, e, &off, &err) && off + h.record_stride > fs + h.record_stride) {
          fprintf(stderr, "record offset past the file\n");
          exit(1);
        }
      }
  } else {
    rejected++;
    if (err.empty()) {
      fprintf(stderr, "rejected without a message\n");
      exit(1);
    }
  }
  return ok;
}

int expect(const std::string& s, bool want, const char* what) {
  if (parse(s) != want) {
    fprintf(stderr, "%s: expected %s for %s\n", what, want ? "accept" : "reject", s.c_str());
    return 1;
  }
  return 0;
}

}  // namespace

int main() {
  int bad = 0;
  bad += expect(VALID, true, "valid header");
  bad += expect("{ \"note\" : {\"a\": [1, 2.5, \"x\\\"y\"], \"b\": null, \"c\": true}, " + VALID.substr(1),
                true, "unknown fields skipped");
  const char* malformed[] = {
      "", "{", "}", "[1,2]", "{\"version\":1", "{\"version\":1,\"dtype\":\"q5_1\"}", "{}",
      "{\"version\":-1}", "{\"version\":1.5}", "{\"version\":99999999999999999999999}",
      "{\"version\":4294967296}", "{\"dtype\":\"q4_0\\", "{\"a\": ,}", "{\"a\":}", "{\"a\"}",
      "{\"moe_layers\":[1,2,]}", "{\"moe_layers\":[", "{\"moe_layers\":[1 2]}", "\"", "{\"",
      "{\"a\":\"\\u12\"", "{,}", "{\"a\":1,}", "{\"a\":1}}"};
  for (const char* m : malformed) bad += expect(m, false, "malformed");
  // missing each field in turn
  const char* fields[] = {"version", "dtype", "hidden_size", "intermediate_size", "num_experts",
                          "moe_layers", "record_bytes", "record_stride", "data_offset"};
  for (const char* f : fields) {
    std::string s = VALID;
    const size_t k = s.find(std::string("\"") + f + "\"");
    s.replace(k + 1, 1, "x");  // renames the key: an unknown field now
    bad += expect(s, false, "missing field");
  }
  // sizes whose file size overflows size_t
  bad += expect("{\"version\":1,\"dtype\":\"q4_0\",\"hidden_size\":64,\"intermediate_size\":32,"
                "\"num_experts\":1099511627776,\"moe_layers\":[0,1],\"record_bytes\":3456,"
                "\"record_stride\":1099511627776,\"data_offset\":16384}",
                false, "overflowing geometry");
  bad += expect("{\"version\":1,\"dtype\":\"q4_0\",\"hidden_size\":64,\"intermediate_size\":32,"
                "\"num_experts\":3,\"moe_layers\":[0],\"record_bytes\":3456,"
                "\"record_stride\":16384,\"data_offset\":18446744073709551615}",
                false, "overflowing data offset");
  // nesting: within the limit, and past it
  bad += expect("{\"n\":" + std::string(60, '[') + std::string(60, ']') + "," + VALID.substr(1), true, "nesting 60");
  bad += expect("{\"n\":" + std::string(100, '[') + std::string(100, ']') + "," + VALID.substr(1), false, "nesting 100");
  bad += expect("{\"n\":" + std::string(100000, '[') , false, "nesting 100000");
  // every truncation of the valid header
  for (size_t n = 0; n < VALID.size(); n++) parse(VALID.substr(0, n));
  // every byte replaced by each structural character
  const char subs[] = {'"', '{', '}', '[', ']', ':', ',', '\\', '0', '9', 'a', ' ', '\0', '\xff', '-', '.'};
  for (size_t i = 0; i < VALID.size(); i++)
    for (char c : subs) {
      std::string s = VALID;
      s[i] = c;
      parse(s);
    }
  // random edits: 1-4 replacements, insertions or deletions
  for (int it = 0; it < 50000; it++) {
    std::string s = VALID;
    const int edits = 1 + (int)(next() % 4);
    for (int e = 0; e < edits; e++) {
      const size_t pos = s.empty() ? 0 : (size_t)(next() % s.size());
      const char c = (char)(next() & 0xff);
      switch (next() % 3) {
        case 0: if (!s.empty()) s[pos] = c; break;
        case 1: s.insert(s.begin() + pos, c); break;
        default: if (!s.empty()) s.erase(pos, 1);
      }
    }
    parse(s);
  }
  // random bytes
  for (int it = 0; it < 5000; it++) {
    std::string s(next() % 300, '\0');
    for (char& c : s) c = (char)(next() & 0xff);
    parse(s);
  }
  printf("%ld %ld\n", accepted, rejected);
  return bad ? 1 : 0;
}
