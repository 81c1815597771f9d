// The LKV2 snapshot format of crates/lumen-mlx/src/kv_disk.rs (host code):
//
//   [4]  magic "LKV2"                       kv_disk.rs:36-40
//   [4]  version u32 LE (2)
//   [4]  manifest_json_len u32 LE
//   [N]  manifest JSON (serde_json of KvManifest, :291-368)
//   [4]  CRC-32 of the JSON bytes
//   [4]  record_count u32 LE
//   records: [1] dtype | [4] ndim | [ndim x 4] shape i32 | [8] data_len u64 |
//            [data_len] bytes | [4] CRC-32 of the record's preceding bytes
//   nothing after the last record                          :371-448
//
// The reader applies the reference's checks in its order (magic, version,
// manifest CRC, manifest fields, then per record: dtype tag, ndim <= 8, no
// negative dimension, data_len equal to what shape x dtype imply, CRC; no
// trailing bytes) and never sizes anything from an unchecked field: it works
// on the caller's bytes in place, so a record's payload must also fit in
// what is left of the input.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace tqkv {
namespace lkv {

constexpr uint32_t kVersion = 2;

// DtypeTag bytes (kv_disk.rs:81-97).
enum Dtype : uint8_t {
  kBool = 0, kU8 = 1, kU16 = 2, kU32 = 3, kU64 = 4, kI8 = 5, kI16 = 6,
  kI32 = 7, kI64 = 8, kF16 = 9, kF32 = 10, kF64 = 11, kBF16 = 12,
};
// Stored bytes per element (stored_elem_size, :72-79); 0 for an unknown tag.
size_t elem_size(uint8_t tag);

// CRC-32 (IEEE 802.3, reflected, the crc32fast crate's), continuing `crc`.
uint32_t crc32(const void* p, size_t n, uint32_t crc = 0);

struct Opt {
  bool has = false;
  uint64_t v = 0;
};

// LayerMeta (kv_disk.rs:291-324); arrays: record indices, -1 for None.
struct Layer {
  std::string kind;  // a LayerKindTag variant name
  uint64_t offset = 0, base_offset = 0;
  std::vector<int64_t> arrays;
  Opt lengths_id, left_padding_id, max_size, keep, idx, bits, qjl_m;
  bool has_group_size = false;
  int64_t group_size = 0;
};

// KvManifest (kv_disk.rs:347-368).
struct Manifest {
  std::string model_fingerprint;
  uint64_t created_at_unix = 0, position = 0;
  std::vector<uint32_t> prefix_tokens;
  Opt last_token;
  bool is_deep = false;
  std::vector<Layer> layers;
};

struct RecordView {
  uint8_t dtype = 0;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  uint64_t bytes = 0;
};

// serde_json::to_vec of the manifest: compact, fields in declaration order,
// None options skipped where the reference skips them.
std::string manifest_json(const Manifest& m);
// serde_json::from_slice into a Manifest (required fields, types, ranges;
// unknown fields ignored, duplicate fields refused).
bool parse_manifest(const char* s, size_t n, Manifest* m, std::string* err);

// read_lkv over an in-memory file.
bool parse(const uint8_t* p, size_t n, Manifest* m, std::vector<RecordView>* recs,
           std::string* err);

// Bytes of a record with `ndim` dimensions and `data_bytes` of payload.
inline uint64_t record_size(size_t ndim, uint64_t data_bytes) {
  return 1 + 4 + 4 * uint64_t(ndim) + 8 + data_bytes + 4;
}
// Bytes of the file header with a manifest of `json_bytes` (up to the record
// count, inclusive).
inline uint64_t header_size(uint64_t json_bytes) { return 4 + 4 + 4 + json_bytes + 4 + 4; }

// Writes the header (magic .. record count) at `out`; returns bytes written.
uint64_t write_header(uint8_t* out, const std::string& json, uint32_t n_records);
// Writes a record's header at `out` (the payload follows it); returns its size.
uint64_t write_record_header(uint8_t* out, uint8_t dtype, const std::vector<int64_t>& shape,
                             uint64_t data_bytes);
// Appends the CRC of the record starting at `rec` whose header and payload
// occupy `len` bytes.
void finish_record(uint8_t* rec, uint64_t len);

}  // namespace lkv
}  // namespace tqkv
