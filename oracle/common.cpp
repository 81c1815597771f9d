// Shared numerics, arrays and digests of the CPU oracle (test infrastructure).
#include "oracle.h"

#include <cstring>
#include <stdexcept>

namespace oracle {

uint16_t f32_to_bf16(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

float bf16_to_f32(uint16_t v) {
  uint32_t b = uint32_t(v) << 16;
  float x;
  std::memcpy(&x, &b, 4);
  return x;
}

// golden_tests.rs:29-35
uint64_t SplitMix64::next() {
  s += 0x9e3779b97f4a7c15ull;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// golden_tests.rs:76-86
void Digest::bytes(const void* p, size_t n) {
  const uint8_t* b = static_cast<const uint8_t*>(p);
  for (size_t i = 0; i < n; ++i) h = (h ^ uint64_t(b[i])) * 0x100000001b3ull;
}

void Digest::num(uint64_t n) {
  uint8_t le[8];
  for (int i = 0; i < 8; ++i) le[i] = uint8_t(n >> (8 * i));
  bytes(le, 8);
}

size_t dtype_size(DType t) {
  switch (t) {
    case DType::U8: return 1;
    case DType::U32: return 4;
    case DType::F32: return 4;
    case DType::BF16: return 2;
  }
  return 0;
}

Arr zeros(DType d, int h, int s, int last) { return Arr(d, h, s, last); }

// MLX/numpy slice semantics: bounds clamp to [0, s], an inverted range is empty.
Arr slice2(const Arr& a, int start, int end) {
  if (start < 0) start = 0;
  if (end > a.s) end = a.s;
  if (end < start) end = start;
  Arr out(a.dt, a.h, end - start, a.last);
  const size_t rb = a.row_bytes();
  for (int hh = 0; hh < a.h; ++hh)
    if (end > start) std::memcpy(out.row(hh, 0), a.row(hh, start), rb * size_t(end - start));
  return out;
}

Arr concat2(const std::vector<const Arr*>& parts) {
  if (parts.empty()) throw std::runtime_error("concat2 of nothing");
  const Arr& p0 = *parts[0];
  int total = 0;
  for (const Arr* p : parts) {
    if (p->dt != p0.dt || p->h != p0.h || p->last != p0.last)
      throw std::runtime_error("concat2 shape mismatch");
    total += p->s;
  }
  Arr out(p0.dt, p0.h, total, p0.last);
  const size_t rb = p0.row_bytes();
  for (int hh = 0; hh < p0.h; ++hh) {
    int at = 0;
    for (const Arr* p : parts) {
      if (p->s) std::memcpy(out.row(hh, at), p->row(hh, 0), rb * size_t(p->s));
      at += p->s;
    }
  }
  return out;
}

void slice_update2(Arr& buf, int start, const Arr& src) {
  if (src.dt != buf.dt || src.h != buf.h || src.last != buf.last || start < 0 ||
      start + src.s > buf.s)
    throw std::runtime_error("slice_update2 shape mismatch");
  const size_t rb = buf.row_bytes();
  for (int hh = 0; hh < buf.h; ++hh)
    if (src.s) std::memcpy(buf.row(hh, start), src.row(hh, 0), rb * size_t(src.s));
}

// golden_tests.rs:88-129: ndim, dims, then (non-empty) a dtype tag and the
// elements; bf16 is widened to f32 bits first.
void digest_array(Digest& d, const Arr& a) {
  d.num(4);
  d.num(1);
  d.num(uint64_t(a.h));
  d.num(uint64_t(a.s));
  d.num(uint64_t(a.last));
  const size_t n = size_t(a.h) * a.s * a.last;
  if (n == 0) return;
  switch (a.dt) {
    case DType::U8:
      d.num(1);
      d.bytes(a.data.data(), n);
      break;
    case DType::U32:
      d.num(2);
      d.bytes(a.data.data(), n * 4);  // little-endian host
      break;
    case DType::F32:
      d.num(3);
      d.bytes(a.data.data(), n * 4);
      break;
    case DType::BF16: {
      d.num(4);
      const uint16_t* p = reinterpret_cast<const uint16_t*>(a.data.data());
      for (size_t i = 0; i < n; ++i) {
        uint32_t w = uint32_t(p[i]) << 16;
        d.bytes(&w, 4);
      }
      break;
    }
  }
}

}  // namespace oracle
