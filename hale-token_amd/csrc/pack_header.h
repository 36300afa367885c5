// pack_header.h -- the Hale expert pack header (src/expert/pack.rs:55-123):
// PackHeader, its JSON reader and record offsets.  Host-only C++.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace hale {

// PackHeader (src/expert/pack.rs:55-73)
struct PackHeader {
  uint32_t version = 0;
  int dtype = -1;
  size_t hidden = 0, inter = 0, num_experts = 0;
  std::vector<size_t> moe_layers;
  size_t record_bytes = 0, record_stride = 0, data_offset = 0;
  // PackHeader::file_size (:96-99); parse_pack_header rejects a header for
  // which it does not fit in size_t, so every record offset fits too
  size_t file_size() const { return data_offset + moe_layers.size() * num_experts * record_stride; }
  bool file_size_checked(size_t* out) const;
};

// Parses the JSON header (serde's PackHeader: fields in any order, unknown
// fields skipped); false with a message on malformed input, a missing
// field or sizes whose file size overflows.
bool parse_pack_header(const char* json, size_t len, PackHeader* h, std::string* err);

// Record offset of (layer, expert); false with a message when the key is
// not in the pack (PackHeader::offset_of, src/expert/pack.rs:104-123).
bool pack_offset_of(const PackHeader& h, uint32_t layer, uint32_t expert, uint64_t* off,
                    std::string* err);

}  // namespace hale
