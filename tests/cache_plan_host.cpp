// TEST HARNESS (not product code). Replays the reference's golden cache plans
// through the product's cache index math (lumen-rs_amd/csrc/cache_plan.hpp)
// with a host-memory executor, folding every fetched view, buffer and counter
// into the FNV-1a digest the way crates/lumen-mlx/src/native_cache/
// golden_tests.rs:236-497 does. The plan inputs and the digest steps come from
// the oracle (oracle_golden_tape, oracle_fnv_*); affine kinds quantize their
// inputs with the oracle's MLX restatement (the device quantizer is checked
// against it separately). A match with the recorded digests pins the
// planner's growth, ring, trim and rewind arithmetic bit for bit.
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "cache_plan.hpp"

extern "C" {
int64_t oracle_golden_tape(const char* kind, const char* plan, int64_t* events,
                           int64_t max_events, uint8_t* data, int64_t data_cap,
                           int64_t* data_len, int64_t* max_size, int64_t* keep);
uint64_t oracle_fnv_num(uint64_t h, uint64_t n);
uint64_t oracle_fnv_array(uint64_t h, int dtype, int hh, int s, int last, const void* data);
void oracle_affine_quantize(const uint16_t* w, size_t rows, int dim, int gs, int bits,
                            uint32_t* packed, uint16_t* scales, uint16_t* biases, int round_mode,
                            int wmax0, int clip_low);
}

namespace {

using namespace tqkv::cacheplan;

constexpr int H = 2;  // golden_tests.rs:273

struct SlotDesc {
  int dtype;  // 1 u8, 2 u32, 3 f32, 4 bf16
  int last;
  int esize() const { return dtype == 1 ? 1 : dtype == 4 ? 2 : 4; }
  int row() const { return last * esize(); }
};

struct Slot {
  SlotDesc d;
  std::vector<uint8_t> buf;  // [H, len, row]
};

std::vector<SlotDesc> slots_of(const std::string& kind) {
  if (kind == "full" || kind == "rot") return {{4, 16}, {4, 24}};
  if (kind == "quant_full" || kind == "rot_quant")
    return {{2, 8}, {4, 1}, {4, 1}, {2, 16}, {4, 2}, {4, 2}};
  if (kind == "tq") return {{1, 16}, {3, 1}, {1, 24}, {3, 1}};
  return {{1, 16}, {3, 1}, {2, 2}, {3, 1}, {1, 24}, {3, 1}};  // tq_qjl
}

// Carry out a plan on one slot: rebuild from pieces, then write `s` new rows
// (`rows`: [H, s, row]) at plan.write_at.
void execute(Slot& sl, int64_t old_len, const Plan& p, const uint8_t* rows, int64_t s) {
  const size_t rb = size_t(sl.d.row());
  std::vector<uint8_t> nb(size_t(H) * p.len * rb, 0);
  for (int h = 0; h < H; ++h) {
    int64_t at = 0;
    for (const Piece& q : p.pieces) {
      if (q.src >= 0)
        std::memcpy(&nb[(size_t(h) * p.len + at) * rb], &sl.buf[(size_t(h) * old_len + q.src) * rb],
                    size_t(q.n) * rb);
      at += q.n;
    }
    std::memcpy(&nb[(size_t(h) * p.len + p.write_at) * rb], rows + size_t(h) * s * rb,
                size_t(s) * rb);
  }
  sl.buf.swap(nb);
}

uint64_t digest_rows(uint64_t d, const Slot& sl, int64_t len, int64_t n) {
  // [1, H, n, last] from the first n rows of each slab of a buffer of len rows
  const size_t rb = size_t(sl.d.row());
  std::vector<uint8_t> v(size_t(H) * n * rb);
  for (int h = 0; h < H; ++h)
    std::memcpy(&v[size_t(h) * n * rb], &sl.buf[size_t(h) * len * rb], size_t(n) * rb);
  return oracle_fnv_array(d, sl.d.dtype, H, int(n), sl.d.last, v.data());
}

}  // namespace

extern "C" uint64_t planhost_golden_digest(const char* kind_c, const char* plan_c, int prealloc) {
  const std::string kind = kind_c;
  std::vector<int64_t> ev(3 * 4096);
  std::vector<uint8_t> data(1 << 24);
  int64_t data_len = 0, max_size = 0, keep = 0;
  const int64_t n_ev = oracle_golden_tape(kind_c, plan_c, ev.data(), 4096, data.data(),
                                          int64_t(data.size()), &data_len, &max_size, &keep);
  if (n_ev < 0) return 0;

  const bool ring = !(kind == "full" || kind == "quant_full");
  const bool quant = kind == "quant_full" || kind == "rot_quant";
  Config cfg;
  cfg.max_size = ring ? max_size : 0;
  cfg.keep = ring ? keep : 0;
  cfg.prealloc = prealloc != 0;
  cfg.quantized = quant;
  State st;
  std::vector<Slot> slots;
  for (const SlotDesc& d : slots_of(kind)) slots.push_back(Slot{d, {}});

  uint64_t d = 0xcbf29ce484222325ull;
  auto opt = [&](const Slot& sl) {
    if (!st.has) {
      d = oracle_fnv_num(d, 0);
    } else {
      d = oracle_fnv_num(d, 1);
      d = digest_rows(d, sl, st.len, st.len);
    }
  };
  auto state = [&]() {
    if (kind == "full") {
      opt(slots[0]);
      opt(slots[1]);
      d = oracle_fnv_num(d, uint64_t(st.offset));
      d = oracle_fnv_num(d, 0);
    } else if (quant) {
      for (int t = 0; t < 2; ++t) {
        if (!st.has) {
          d = oracle_fnv_num(d, 0);
          continue;
        }
        d = oracle_fnv_num(d, 1);
        for (int i = 0; i < 3; ++i) d = digest_rows(d, slots[3 * t + i], st.len, st.len);
      }
      d = oracle_fnv_num(d, uint64_t(st.offset));
    } else if (kind == "rot") {
      opt(slots[0]);
      opt(slots[1]);
    } else if (kind == "tq") {
      for (int i = 0; i < 4; ++i) opt(slots[i]);
      d = oracle_fnv_num(d, 0);
      d = oracle_fnv_num(d, 0);
    } else {
      const int order[6] = {0, 1, 4, 5, 2, 3};
      for (int i : order) opt(slots[i]);
    }
    if (ring) {
      if (kind == "rot_quant") {
        // quant branch above already folded the triples and the offset
        d = oracle_fnv_num(d, uint64_t(st.idx));
        d = oracle_fnv_num(d, uint64_t(st.has ? st.len : 0));
      } else {
        d = oracle_fnv_num(d, uint64_t(st.offset));
        d = oracle_fnv_num(d, uint64_t(st.idx));
        d = oracle_fnv_num(d, uint64_t(st.has ? st.len : 0));
      }
    }
  };

  for (int64_t e = 0; e < n_ev; ++e) {
    const char op = char(ev[3 * e]);
    const int64_t n = ev[3 * e + 1], at = ev[3 * e + 2];
    if (op == 'R') {
      d = oracle_fnv_num(d, truncate(st, cfg, n) ? 1 : 0);
      state();
      continue;
    }
    const int64_t s = n;
    // The update's rows per slot, [H, s, row].
    std::vector<std::vector<uint8_t>> rows(slots.size());
    const uint8_t* p = data.data() + at;
    if (quant) {
      for (int t = 0; t < 2; ++t) {
        const int dim = t == 0 ? 64 : 128;
        const size_t rws = size_t(H) * s;
        std::vector<uint32_t> pk(rws * dim * 4 / 32);
        std::vector<uint16_t> sc(rws * dim / 64), bi(rws * dim / 64);
        oracle_affine_quantize(reinterpret_cast<const uint16_t*>(p), rws, dim, 64, 4, pk.data(),
                               sc.data(), bi.data(), 0, 1, 0);
        p += rws * dim * 2;
        rows[3 * t].assign(reinterpret_cast<uint8_t*>(pk.data()),
                           reinterpret_cast<uint8_t*>(pk.data()) + pk.size() * 4);
        rows[3 * t + 1].assign(reinterpret_cast<uint8_t*>(sc.data()),
                               reinterpret_cast<uint8_t*>(sc.data()) + sc.size() * 2);
        rows[3 * t + 2].assign(reinterpret_cast<uint8_t*>(bi.data()),
                               reinterpret_cast<uint8_t*>(bi.data()) + bi.size() * 2);
      }
    } else {
      for (size_t i = 0; i < slots.size(); ++i) {
        const size_t nb = size_t(H) * s * slots[i].d.row();
        rows[i].assign(p, p + nb);
        p += nb;
      }
    }
    const int64_t old_len = st.has ? st.len : 0;
    const Plan plan = update(st, cfg, s);
    for (size_t i = 0; i < slots.size(); ++i) execute(slots[i], old_len, plan, rows[i].data(), s);
    // fetched views
    if (quant) {
      for (int t = 0; t < 2; ++t) {
        d = oracle_fnv_num(d, 1);
        for (int i = 0; i < 3; ++i) d = digest_rows(d, slots[3 * t + i], st.len, plan.view);
      }
    } else {
      for (const Slot& sl : slots) d = digest_rows(d, sl, st.len, plan.view);
    }
    state();
  }
  return d;
}
