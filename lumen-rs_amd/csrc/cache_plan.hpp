// Index math of the KV caches, as plain C++ (no HIP): what a cache update
// does to its buffers, expressed as a plan that an executor carries out on
// device memory (cache.hip) or, in the tests, on host memory.
//
// A cache holds parallel buffers ("slots": keys, values, and for quantized
// formats their scales and biases), all with the same token length; every
// update moves them together. The reference keeps each slot as an MLX array
// [B, H_kv, len, row] that its updates replace by slices and
// concatenations; here a slot is one allocation with a row capacity and a
// logical length, and an update is
//   1. the new buffer as a concatenation of pieces: row ranges of the old
//      buffer and runs of zero rows (often just "the old buffer, then zeros"),
//   2. the update's S new rows written at one row position,
// after which the fetched view is the first `view` rows.
//
// The arithmetic follows crates/lumen-mlx/src/native_cache.rs:
//   step-256 growth (update_and_fetch :591-736, KV_CACHE_STEP :37, truncate
//   :778-811, quantized :913-1119), the rotating buffer's in-place write
//   (ring_update_in_place :146-231), its concatenating path
//   (rotating_concat :86-125, ring_update_concat :240-268, dispatch
//   ring_update :277-290) and its rewind (ring_truncate :304-335).
#pragma once

#include <cstdint>
#include <vector>

namespace tqkv {
namespace cacheplan {

constexpr int64_t kStep = 256;  // native_cache.rs:37

// A piece of the new buffer: rows [src, src + n) of the old buffer, or
// (src < 0) n zero rows.
struct Piece {
  int64_t src;
  int64_t n;
};

struct Plan {
  std::vector<Piece> pieces;  // the new buffer, in order
  int64_t len = 0;            // its length (sum of the pieces)
  int64_t write_at = 0;       // where the S new rows go
  int64_t view = 0;           // rows of the fetched view
  // true when the new buffer keeps rows [0, old_len) in place and only
  // appends zeros (or nothing): the executor can grow it in place.
  bool keeps_prefix(int64_t old_len) const {
    int64_t at = 0;
    for (const Piece& p : pieces) {
      if (p.src >= 0) {
        if (p.src != at) return false;
        at += p.n;
      } else {
        return at == old_len;
      }
    }
    return at == old_len;
  }
};

struct State {
  bool has = false;      // buffers exist (the reference's Option<Array>)
  int64_t len = 0;       // buffer length (cached_len)
  int64_t offset = 0;    // tokens seen (the reference's offset)
  int64_t idx = 0;       // ring write position
};

struct Config {
  int64_t max_size = 0;  // > 0: rotating window of this many tokens
  int64_t keep = 0;      // ring: sink tokens kept at the head
  bool prealloc = true;  // LUMEN_NATIVE_KV_STEP_PREALLOC
  bool quantized = false;  // affine caches refuse rewinds on the legacy path
};

inline void push(Plan& p, int64_t src, int64_t n) {
  if (n <= 0) return;
  if (!p.pieces.empty()) {
    Piece& b = p.pieces.back();
    if (src < 0 && b.src < 0) {
      b.n += n;
      p.len += n;
      return;
    }
    if (src >= 0 && b.src >= 0 && b.src + b.n == src) {
      b.n += n;
      p.len += n;
      return;
    }
  }
  p.pieces.push_back(Piece{src, n});
  p.len += n;
}

// Rows [a, b) of a concatenation of pieces, as pieces.
inline std::vector<Piece> slice(const std::vector<Piece>& ps, int64_t a, int64_t b) {
  std::vector<Piece> out;
  int64_t at = 0;
  for (const Piece& p : ps) {
    const int64_t lo = a > at ? a : at, hi = b < at + p.n ? b : at + p.n;
    if (lo < hi) out.push_back(Piece{p.src < 0 ? -1 : p.src + (lo - at), hi - lo});
    at += p.n;
  }
  return out;
}

// Growing cache (NativeKvCache / NativeKvCacheQuantized), S new rows.
inline Plan step_update(State& st, const Config& c, int64_t s) {
  Plan p;
  const int64_t prev = st.offset, total = prev + s;
  if (!c.prealloc) {
    // legacy path: concatenate onto the whole buffer
    if (st.has) push(p, 0, st.len);
    p.write_at = p.len;
    push(p, -1, s);
    p.view = p.len;
  } else {
    if (!st.has || total > st.len) {
      const int64_t n_steps = (kStep + s - 1) / kStep;
      if (st.has) push(p, 0, (prev % kStep != 0) ? prev : st.len);
      push(p, -1, n_steps * kStep);
    } else {
      push(p, 0, st.len);
    }
    p.write_at = prev;
    p.view = total;
  }
  st.has = true;
  st.len = p.len;
  st.offset = total;
  return p;
}

// Rotating cache, one token written in place (S == 1 with prealloc).
inline Plan ring_in_place(State& st, const Config& c) {
  Plan p;
  const int64_t prev = st.offset;
  int64_t len = st.has ? st.len : 0;
  std::vector<Piece> buf;
  if (st.has) buf.push_back(Piece{0, len});
  const bool need_grow = !st.has || (prev >= len && len < c.max_size);
  if (need_grow) {
    const int64_t grow = kStep < c.max_size - prev ? kStep : c.max_size - prev;
    buf.push_back(Piece{-1, grow});
    len += grow;
    st.idx = prev;
  }
  if (len > c.max_size) {
    const int64_t trim = len - c.max_size;
    std::vector<Piece> head = slice(buf, 0, c.keep), tail = slice(buf, trim + c.keep, len);
    buf = head;
    buf.insert(buf.end(), tail.begin(), tail.end());
    len = c.max_size;
    st.idx = c.max_size;
  }
  if (st.idx == c.max_size) st.idx = c.keep;
  for (const Piece& q : buf) push(p, q.src, q.n);
  p.write_at = st.idx;
  st.idx += 1;
  st.offset = prev + 1;
  st.has = true;
  st.len = p.len;
  p.view = st.offset >= c.max_size ? p.len : st.offset;
  return p;
}

// Rotating cache, S rows by concatenation (rotating_concat).
inline Plan ring_concat(State& st, const Config& c, int64_t s) {
  Plan p;
  if (!st.has) {
    push(p, -1, s);
  } else {
    const int64_t len = st.len;
    std::vector<Piece> ordered;
    if (st.idx == len) {
      ordered = {Piece{0, len}};
    } else if (st.idx < st.offset) {
      ordered = {Piece{0, c.keep}, Piece{st.idx, len - st.idx}, Piece{c.keep, st.idx - c.keep}};
    } else {
      ordered = {Piece{0, st.idx}};
    }
    int64_t held = 0;
    for (const Piece& q : ordered) held += q.n;
    const int64_t trim = held + 1 > c.max_size ? held + 1 - c.max_size : 0;
    std::vector<Piece> kept = ordered;
    if (trim > 0) {
      kept = slice(ordered, 0, c.keep);
      std::vector<Piece> tail = slice(ordered, trim + c.keep, held);
      kept.insert(kept.end(), tail.begin(), tail.end());
    }
    for (const Piece& q : kept) push(p, q.src, q.n);
    push(p, -1, s);
  }
  p.write_at = p.len - s;
  p.view = p.len;
  st.offset += s;
  st.idx = p.len;
  st.has = true;
  st.len = p.len;
  return p;
}

inline Plan ring_update(State& st, const Config& c, int64_t s) {
  if (s == 1 && c.prealloc) return ring_in_place(st, c);
  return ring_concat(st, c, s);
}

inline Plan update(State& st, const Config& c, int64_t s) {
  return c.max_size > 0 ? ring_update(st, c, s) : step_update(st, c, s);
}

// Rewind to `target` tokens. false = the reference's Err: a target past the
// offset; for a ring, any rewind once it has wrapped (offset > max_size);
// for a quantized growing cache, any real rewind on the legacy path.
inline bool truncate(State& st, const Config& c, int64_t target) {
  if (target < 0 || target > st.offset) return false;
  if (target == st.offset) return true;
  if (c.max_size > 0) {
    if (st.offset > c.max_size) return false;
    st.offset = target;
    st.idx = target;
    return true;
  }
  if (c.quantized && !c.prealloc) return false;
  st.offset = target;
  return true;
}

}  // namespace cacheplan
}  // namespace tqkv
