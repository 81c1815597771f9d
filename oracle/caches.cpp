// Every KV-cache kind of native_cache.rs restated over host arrays, and the
// reference's golden plans replayed into FNV-1a digests (test infrastructure).
//
// The digests the reference recorded (golden_tests.rs:413-497) fold in every
// fetched view, every backing buffer (zero padding and stale slots included)
// and every counter after every step, so matching them pins the growth,
// ring-rotation, trim and rewind arithmetic bit for bit.
#include <algorithm>
#include <memory>
#include <optional>
#include <stdexcept>

#include "oracle.h"

namespace oracle {
namespace {

constexpr size_t kStep = 256;  // native_cache.rs:37 KV_CACHE_STEP

using Slot = std::optional<Arr>;

// ------------------------------------------------------------ ring helpers
// native_cache.rs:86-125
Arr rotating_concat(const Arr& old, const Arr& nw, size_t idx, size_t offset, size_t keep,
                    size_t max_size) {
  const size_t buf = size_t(old.s);
  Arr ordered;
  if (idx == buf) {
    ordered = old;
  } else if (idx < offset) {
    Arr a = slice2(old, 0, int(keep)), b = slice2(old, int(idx), int(buf)),
        c = slice2(old, int(keep), int(idx));
    ordered = concat2({&a, &b, &c});
  } else {
    ordered = slice2(old, 0, int(idx));
  }
  const size_t held = size_t(ordered.s);
  const size_t trim = held + 1 > max_size ? held + 1 - max_size : 0;
  if (trim == 0) return concat2({&ordered, &nw});
  Arr a = slice2(ordered, 0, int(keep)), b = slice2(ordered, int(trim + keep), int(held));
  return concat2({&a, &b, &nw});
}

// native_cache.rs:146-231
std::vector<Arr> ring_update_in_place(std::vector<Slot*> bufs, std::vector<const Arr*> nw,
                                      size_t& offset, size_t& idx, size_t max_size,
                                      size_t keep) {
  const size_t prev = offset;
  const bool need_grow = !bufs[0]->has_value() ||
                         (prev >= size_t((*bufs[0])->s) && size_t((*bufs[0])->s) < max_size);
  if (need_grow) {
    const size_t new_size = std::min(kStep, max_size - prev);
    for (size_t i = 0; i < bufs.size(); ++i) {
      Arr block = zeros(nw[i]->dt, nw[i]->h, int(new_size), nw[i]->last);
      if (!bufs[i]->has_value())
        *bufs[i] = block;
      else
        *bufs[i] = concat2({&**bufs[i], &block});
    }
    idx = prev;
  }
  const size_t buf_size = size_t((*bufs[0])->s);
  if (buf_size > max_size) {
    const size_t trim = buf_size - max_size;
    for (Slot* b : bufs) {
      Arr a = slice2(**b, 0, int(keep)), c = slice2(**b, int(trim + keep), int(buf_size));
      *b = concat2({&a, &c});
    }
    idx = max_size;
  }
  if (idx == max_size) idx = keep;
  for (size_t i = 0; i < bufs.size(); ++i) slice_update2(**bufs[i], int(idx), *nw[i]);
  idx += 1;
  offset = prev + 1;
  std::vector<Arr> fetched;
  for (Slot* b : bufs)
    fetched.push_back(offset >= max_size ? **b : slice2(**b, 0, int(offset)));
  return fetched;
}

// native_cache.rs:240-268
std::vector<Arr> ring_update_concat(std::vector<Slot*> bufs, std::vector<const Arr*> nw,
                                    size_t& offset, size_t& idx, size_t max_size,
                                    size_t keep) {
  std::vector<Arr> fetched;
  for (size_t i = 0; i < bufs.size(); ++i) {
    if (!bufs[i]->has_value())
      fetched.push_back(*nw[i]);
    else
      fetched.push_back(rotating_concat(**bufs[i], *nw[i], idx, offset, keep, max_size));
  }
  offset += size_t(nw[0]->s);
  idx = size_t(fetched[0].s);
  for (size_t i = 0; i < bufs.size(); ++i) *bufs[i] = fetched[i];
  return fetched;
}

// native_cache.rs:277-290
std::vector<Arr> ring_update(std::vector<Slot*> bufs, std::vector<const Arr*> nw,
                             size_t& offset, size_t& idx, size_t max_size, size_t keep,
                             bool prealloc) {
  if (nw[0]->s == 1 && prealloc)
    return ring_update_in_place(bufs, nw, offset, idx, max_size, keep);
  return ring_update_concat(bufs, nw, offset, idx, max_size, keep);
}

// native_cache.rs:304-335 (Ok -> true, Err -> false)
bool ring_truncate(size_t& offset, size_t& idx, size_t max_size, size_t target) {
  if (target > offset) return false;
  if (target == offset) return true;
  if (offset > max_size) return false;
  offset = target;
  idx = target;
  return true;
}

// ------------------------------------------------------------ golden inputs
// golden_tests.rs:37-65
struct Inputs {
  SplitMix64 rng;
  explicit Inputs(uint64_t seed) : rng(seed) {}
  Arr bf16(int h, int s, int d) {
    Arr a(DType::BF16, h, s, d);
    uint16_t* p = reinterpret_cast<uint16_t*>(a.data.data());
    for (size_t i = 0; i < size_t(h) * s * d; ++i) {
      float f = float(rng.next() >> 40) / float(1u << 22) - 2.0f;
      p[i] = f32_to_bf16(f);
    }
    return a;
  }
  Arr positive(int h, int s, int d) {
    Arr a(DType::F32, h, s, d);
    float* p = reinterpret_cast<float*>(a.data.data());
    for (size_t i = 0; i < size_t(h) * s * d; ++i)
      p[i] = float(rng.next() >> 40) / float(1u << 24) + 0.5f;
    return a;
  }
  Arr codes(int h, int s, int d) {
    Arr a(DType::U8, h, s, d);
    for (size_t i = 0; i < size_t(h) * s * d; ++i) a.data[i] = uint8_t(rng.next() >> 60);
    return a;
  }
  Arr words(int h, int s, int d) {
    Arr a(DType::U32, h, s, d);
    uint32_t* p = reinterpret_cast<uint32_t*>(a.data.data());
    for (size_t i = 0; i < size_t(h) * s * d; ++i) p[i] = uint32_t(rng.next());
    return a;
  }
};

void digest_opt(Digest& d, const Slot& s) {
  if (s.has_value()) {
    d.num(1);
    digest_array(d, *s);
  } else {
    d.num(0);
  }
}

// An affine triple (packed u32, scales bf16, biases bf16) of bf16 input x.
struct Triple {
  Arr w, s, b;
};
Triple quantize(const Arr& x, int gs, int bits, const AffineOpts& ao) {
  const size_t rows = size_t(x.h) * x.s;
  Triple t{Arr(DType::U32, x.h, x.s, x.last * bits / 32), Arr(DType::BF16, x.h, x.s, x.last / gs),
           Arr(DType::BF16, x.h, x.s, x.last / gs)};
  affine_quantize_rows(reinterpret_cast<const uint16_t*>(x.data.data()), rows, x.last, gs, bits,
                       reinterpret_cast<uint32_t*>(t.w.data.data()),
                       reinterpret_cast<uint16_t*>(t.s.data.data()),
                       reinterpret_cast<uint16_t*>(t.b.data.data()), ao);
  return t;
}

// ------------------------------------------------------------ cache kinds
struct Case {
  virtual ~Case() = default;
  virtual void update(int s, Inputs& in, Digest& d) = 0;
  virtual bool rewind(size_t target) = 0;
  virtual void state(Digest& d) const = 0;
};

constexpr int H = 2;  // golden_tests.rs:273

// NativeKvCache, native_cache.rs:591-736 (update) and :778-811 (truncate).
// It also serves as a step-256 allocator model for several buffers at once:
// `bufs` move together, buffer 0 decides growth.
struct StepBuffers {
  std::vector<Slot> bufs;
  size_t offset = 0;
  explicit StepBuffers(size_t n) : bufs(n) {}
  std::vector<Arr> update(const std::vector<const Arr*>& nw, bool prealloc) {
    const size_t s = size_t(nw[0]->s), prev = offset, total = prev + s;
    if (!prealloc) {
      for (size_t i = 0; i < bufs.size(); ++i)
        bufs[i] = bufs[i].has_value() ? concat2({&*bufs[i], nw[i]}) : *nw[i];
      offset = total;
      std::vector<Arr> out;
      for (auto& b : bufs) out.push_back(*b);
      return out;
    }
    if (!bufs[0].has_value() || total > size_t(bufs[0]->s)) {
      const size_t n_steps = (kStep + s - 1) / kStep;
      for (size_t i = 0; i < bufs.size(); ++i) {
        Arr block = zeros(nw[i]->dt, nw[i]->h, int(n_steps * kStep), nw[i]->last);
        if (!bufs[i].has_value()) {
          bufs[i] = block;
        } else {
          Arr kept = (prev % kStep != 0) ? slice2(*bufs[i], 0, int(prev)) : *bufs[i];
          bufs[i] = concat2({&kept, &block});
        }
      }
    }
    for (size_t i = 0; i < bufs.size(); ++i) slice_update2(*bufs[i], int(prev), *nw[i]);
    offset = total;
    std::vector<Arr> out;
    for (auto& b : bufs) out.push_back(slice2(*b, 0, int(total)));
    return out;
  }
};

struct FullCase : Case {
  StepBuffers sb{2};
  bool prealloc;
  explicit FullCase(bool p) : prealloc(p) {}
  void update(int s, Inputs& in, Digest& d) override {
    Arr k = in.bf16(H, s, 16), v = in.bf16(H, s, 24);
    auto f = sb.update({&k, &v}, prealloc);
    digest_array(d, f[0]);
    digest_array(d, f[1]);
  }
  bool rewind(size_t target) override {
    if (target > sb.offset) return false;
    sb.offset = target;
    return true;
  }
  void state(Digest& d) const override {
    digest_opt(d, sb.bufs[0]);
    digest_opt(d, sb.bufs[1]);
    d.num(sb.offset);
    d.num(0);  // base_offset
  }
};

// NativeKvCacheQuantized, native_cache.rs:913-1119
struct QuantFullCase : Case {
  StepBuffers sb{6};
  bool prealloc;
  AffineOpts ao;
  QuantFullCase(bool p, const AffineOpts& o) : prealloc(p), ao(o) {}
  void update(int s, Inputs& in, Digest& d) override {
    Arr k = in.bf16(H, s, 64), v = in.bf16(H, s, 128);
    Triple kt = quantize(k, 64, 4, ao), vt = quantize(v, 64, 4, ao);
    auto f = sb.update({&kt.w, &kt.s, &kt.b, &vt.w, &vt.s, &vt.b}, prealloc);
    for (int t = 0; t < 2; ++t) {
      d.num(1);
      for (int i = 0; i < 3; ++i) digest_array(d, f[3 * t + i]);
    }
  }
  bool rewind(size_t target) override {
    if (target > sb.offset) return false;
    if (target == sb.offset) return true;
    if (!prealloc) return false;
    sb.offset = target;
    return true;
  }
  void state(Digest& d) const override {
    for (int t = 0; t < 2; ++t) {
      if (!sb.bufs[3 * t].has_value()) {
        d.num(0);
        continue;
      }
      d.num(1);
      for (int i = 0; i < 3; ++i) digest_array(d, *sb.bufs[3 * t + i]);
    }
    d.num(sb.offset);
  }
};

// Rotating caches over N parallel buffers (native_cache.rs:1145-1862).
struct RingCase : Case {
  std::vector<Slot> bufs;
  size_t offset = 0, idx = 0, max_size, keep;
  bool prealloc;
  RingCase(size_t n, size_t mx, size_t kp, bool p) : bufs(n), max_size(mx), keep(kp), prealloc(p) {}
  std::vector<Arr> push(const std::vector<const Arr*>& nw) {
    std::vector<Slot*> ptrs;
    for (auto& b : bufs) ptrs.push_back(&b);
    return ring_update(ptrs, nw, offset, idx, max_size, keep, prealloc);
  }
  bool rewind(size_t target) override { return ring_truncate(offset, idx, max_size, target); }
  size_t cached_len() const { return bufs[0].has_value() ? size_t(bufs[0]->s) : 0; }
};

struct RotCase : RingCase {
  RotCase(size_t mx, size_t kp, bool p) : RingCase(2, mx, kp, p) {}
  void update(int s, Inputs& in, Digest& d) override {
    Arr k = in.bf16(H, s, 16), v = in.bf16(H, s, 24);
    auto f = push({&k, &v});
    digest_array(d, f[0]);
    digest_array(d, f[1]);
  }
  void state(Digest& d) const override {
    digest_opt(d, bufs[0]);
    digest_opt(d, bufs[1]);
    d.num(offset);
    d.num(idx);
    d.num(cached_len());
  }
};

struct RotQuantCase : RingCase {
  AffineOpts ao;
  RotQuantCase(size_t mx, size_t kp, bool p, const AffineOpts& o) : RingCase(6, mx, kp, p), ao(o) {}
  void update(int s, Inputs& in, Digest& d) override {
    Arr k = in.bf16(H, s, 64), v = in.bf16(H, s, 128);
    Triple kt = quantize(k, 64, 4, ao), vt = quantize(v, 64, 4, ao);
    auto f = push({&kt.w, &kt.s, &kt.b, &vt.w, &vt.s, &vt.b});
    for (int t = 0; t < 2; ++t) {
      d.num(1);
      for (int i = 0; i < 3; ++i) digest_array(d, f[3 * t + i]);
    }
  }
  void state(Digest& d) const override {
    for (int t = 0; t < 2; ++t) {
      if (!bufs[3 * t].has_value()) {
        d.num(0);
        continue;
      }
      d.num(1);
      for (int i = 0; i < 3; ++i) digest_array(d, *bufs[3 * t + i]);
    }
    d.num(offset);
    d.num(idx);
    d.num(cached_len());
  }
};

// NativeRotatingKvCacheTurboQuant: slots kc, ks, vc, vs (+ ksg, krn with QJL).
struct TqCase : RingCase {
  bool qjl;
  TqCase(size_t mx, size_t kp, bool p, bool q) : RingCase(q ? 6 : 4, mx, kp, p), qjl(q) {}
  void update(int s, Inputs& in, Digest& d) override {
    if (!qjl) {
      Arr kc = in.codes(H, s, 16), ks = in.positive(H, s, 1);
      Arr vc = in.codes(H, s, 24), vs = in.positive(H, s, 1);
      auto f = push({&kc, &ks, &vc, &vs});
      for (auto& a : f) digest_array(d, a);
    } else {
      Arr kc = in.codes(H, s, 16), ks = in.positive(H, s, 1);
      Arr ksg = in.words(H, s, 2), krn = in.positive(H, s, 1);
      Arr vc = in.codes(H, s, 24), vs = in.positive(H, s, 1);
      auto f = push({&kc, &ks, &ksg, &krn, &vc, &vs});
      for (auto& a : f) digest_array(d, a);
    }
  }
  void state(Digest& d) const override {
    // turboquant_state order (golden_tests.rs:361-371): kc, ks, vc, vs, signs, rnorm
    if (!qjl) {
      for (int i = 0; i < 4; ++i) digest_opt(d, bufs[i]);
      d.num(0);
      d.num(0);
    } else {
      const int order[6] = {0, 1, 4, 5, 2, 3};
      for (int i : order) digest_opt(d, bufs[i]);
    }
    d.num(offset);
    d.num(idx);
    d.num(cached_len());
  }
};

// ------------------------------------------------------------ plans
struct Step {
  char op;  // 'C' chunk, 'D' decode, 'R' rewind
  size_t n;
};
// golden_tests.rs:182-226
const std::vector<Step> kFull = {{'D', 3},   {'C', 250}, {'D', 5}, {'C', 300}, {'R', 500},
                                 {'D', 3},   {'R', 600}, {'C', 7}, {'R', 510}, {'D', 2}};
const std::vector<Step> kSmallRing = {{'C', 5},  {'D', 3},  {'R', 6}, {'D', 4},
                                      {'C', 3},  {'D', 10}, {'C', 20}, {'D', 5},
                                      {'R', 30}, {'C', 4},  {'D', 3}};
const std::vector<Step> kLargeRing = {{'D', 3},  {'R', 2}, {'C', 260}, {'D', 40},
                                      {'C', 30}, {'D', 3}, {'R', 50},  {'C', 2}};

// golden_tests.rs:236-256
uint64_t run(Case& c, const std::vector<Step>& steps) {
  Inputs in(0x0022dedcull);
  Digest d;
  for (const Step& st : steps) {
    size_t times = st.op == 'D' ? st.n : 1;
    for (size_t t = 0; t < times; ++t) {
      if (st.op == 'R')
        d.num(c.rewind(st.n) ? 1 : 0);
      else
        c.update(st.op == 'D' ? 1 : int(st.n), in, d);
      c.state(d);
    }
  }
  return d.h;
}

}  // namespace

uint64_t golden_digest(const std::string& kind, const std::string& plan, bool prealloc,
                       const AffineOpts& ao) {
  const std::vector<Step>* steps;
  size_t max_size = 0, keep = 0;
  if (plan == "full") {
    steps = &kFull;
    max_size = 4096;
    keep = 0;
  } else if (plan == "small") {
    steps = &kSmallRing;
    max_size = 12;
    keep = 2;
  } else if (plan == "large") {
    steps = &kLargeRing;
    max_size = 300;
    keep = 4;
  } else {
    throw std::runtime_error("unknown plan " + plan);
  }
  std::unique_ptr<Case> c;
  if (kind == "full")
    c.reset(new FullCase(prealloc));
  else if (kind == "quant_full")
    c.reset(new QuantFullCase(prealloc, ao));
  else if (kind == "rot")
    c.reset(new RotCase(max_size, keep, prealloc));
  else if (kind == "rot_quant")
    c.reset(new RotQuantCase(max_size, keep, prealloc, ao));
  else if (kind == "tq")
    c.reset(new TqCase(max_size, keep, prealloc, false));
  else if (kind == "tq_qjl")
    c.reset(new TqCase(max_size, keep, prealloc, true));
  else
    throw std::runtime_error("unknown kind " + kind);
  return run(*c, *steps);
}

// The inputs a golden plan feeds its cache, in order, without running the
// cache: events (op, n) and, for each update, its arrays as generated
// (golden_tests.rs:37-65 generators, :236-256 driver). Lets another
// implementation of the caches replay exactly the reference's recordings.
GoldenTape golden_tape(const std::string& kind, const std::string& plan) {
  GoldenTape t;
  const std::vector<Step>* steps;
  if (plan == "full") {
    steps = &kFull;
    t.max_size = 4096;
    t.keep = 0;
  } else if (plan == "small") {
    steps = &kSmallRing;
    t.max_size = 12;
    t.keep = 2;
  } else if (plan == "large") {
    steps = &kLargeRing;
    t.max_size = 300;
    t.keep = 4;
  } else {
    throw std::runtime_error("unknown plan " + plan);
  }
  Inputs in(0x0022dedcull);
  auto put = [&](const Arr& a) { t.data.insert(t.data.end(), a.data.begin(), a.data.end()); };
  for (const Step& st : *steps) {
    const size_t times = st.op == 'D' ? st.n : 1;
    for (size_t r = 0; r < times; ++r) {
      const int s = st.op == 'D' ? 1 : int(st.n);
      t.events.push_back({st.op == 'R' ? 'R' : 'U', st.op == 'R' ? int64_t(st.n) : int64_t(s),
                          int64_t(t.data.size())});
      if (st.op == 'R') continue;
      if (kind == "full" || kind == "rot") {
        put(in.bf16(H, s, 16));
        put(in.bf16(H, s, 24));
      } else if (kind == "quant_full" || kind == "rot_quant") {
        put(in.bf16(H, s, 64));
        put(in.bf16(H, s, 128));
      } else if (kind == "tq") {
        put(in.codes(H, s, 16));
        put(in.positive(H, s, 1));
        put(in.codes(H, s, 24));
        put(in.positive(H, s, 1));
      } else if (kind == "tq_qjl") {
        put(in.codes(H, s, 16));
        put(in.positive(H, s, 1));
        put(in.words(H, s, 2));
        put(in.positive(H, s, 1));
        put(in.codes(H, s, 24));
        put(in.positive(H, s, 1));
      } else {
        throw std::runtime_error("unknown kind " + kind);
      }
    }
  }
  return t;
}

bool mask_allowed(size_t q_abs, size_t k_abs, long window) {
  if (!(q_abs >= k_abs)) return false;
  if (window >= 0 && !(q_abs < k_abs + size_t(window))) return false;
  return true;
}

}  // namespace oracle
