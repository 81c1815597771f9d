// Host-only driver for the LKV2 reader and writer under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/test_lkv_sanitize.py with the
// sanitizers on the host pass only). It runs the fault sweeps of the
// reference's crates/lumen-mlx/tests/kv_disk_faults.rs over each snapshot
// named on the command line, plus a seeded mutation sweep, with every input
// in a heap block of exactly its own size so a read one byte past the end is
// reported. A sanitizer report aborts the process; the Python side checks the
// exit status and the summary line.
//
// Usage: lkv_sanitize <snapshot>... ; a file whose name ends in ".bad" must be
// rejected as it stands, any other must read.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "tqkv.h"

namespace {

long g_calls = 0;

// The bytes in a heap block of exactly n bytes (n = 0 gives a 1-byte block
// that the callee is told holds nothing).
struct Exact {
  uint8_t* p;
  size_t n;
  Exact(const uint8_t* src, size_t n_) : p(static_cast<uint8_t*>(malloc(n_ ? n_ : 1))), n(n_) {
    if (n) memcpy(p, src, n);
  }
  ~Exact() { free(p); }
  Exact(const Exact&) = delete;
  Exact& operator=(const Exact&) = delete;
};

// Every entry that reads a snapshot, on one input. Returns the check status;
// the other entries must agree with it, and a snapshot that reads must
// rewrite to one that reads again and rewrites to itself.
int32_t exercise(const uint8_t* src, size_t n) {
  Exact in(src, n);
  ++g_calls;
  const int32_t rc = tqkv_lkv_check(in.p, in.n);
  size_t json_bytes = 0;
  int32_t n_layers = -1, n_records = -1;
  const int32_t rm = tqkv_lkv_manifest(in.p, in.n, nullptr, 0, &json_bytes, &n_layers, &n_records);
  size_t out_bytes = 0;
  const int32_t rw = tqkv_lkv_rewrite(in.p, in.n, nullptr, 0, &out_bytes);
  if (rm != rc || rw != rc) {
    fprintf(stderr, "entries disagree: check %d manifest %d rewrite %d\n", rc, rm, rw);
    exit(3);
  }
  if (rc != TQKV_OK) return rc;
  // The manifest into a buffer one byte short (refused), then exactly sized.
  std::vector<char> js(json_bytes + 1);
  if (json_bytes && tqkv_lkv_manifest(in.p, in.n, js.data(), json_bytes, nullptr, nullptr,
                                      nullptr) == TQKV_OK) {
    fprintf(stderr, "manifest accepted a short buffer\n");
    exit(3);
  }
  if (tqkv_lkv_manifest(in.p, in.n, js.data(), js.size(), nullptr, nullptr, nullptr) != TQKV_OK ||
      js[json_bytes] != '\0') {
    fprintf(stderr, "manifest copy failed\n");
    exit(3);
  }
  uint8_t* buf = static_cast<uint8_t*>(malloc(out_bytes ? out_bytes : 1));
  size_t got = 0;
  if (out_bytes && tqkv_lkv_rewrite(in.p, in.n, buf, out_bytes - 1, &got) == TQKV_OK) {
    fprintf(stderr, "rewrite accepted a short buffer\n");
    exit(3);
  }
  if (tqkv_lkv_rewrite(in.p, in.n, buf, out_bytes, &got) != TQKV_OK || got != out_bytes ||
      tqkv_lkv_check(buf, got) != TQKV_OK) {
    fprintf(stderr, "rewrite of a good snapshot does not read: %s\n", tqkv_last_error());
    exit(3);
  }
  Exact again(buf, got);
  free(buf);
  std::vector<uint8_t> twice(got);
  size_t got2 = 0;
  if (tqkv_lkv_rewrite(again.p, again.n, twice.data(), twice.size(), &got2) != TQKV_OK ||
      got2 != got || memcmp(twice.data(), again.p, got) != 0) {
    fprintf(stderr, "rewrite is not idempotent\n");
    exit(3);
  }
  return rc;
}

void expect_corrupt(const std::vector<uint8_t>& d, const char* what, size_t at) {
  const int32_t rc = exercise(d.data(), d.size());
  if (rc != TQKV_ECORRUPT) {
    fprintf(stderr, "%s at %zu of %zu: status %d, want %d\n", what, at, d.size(), rc,
            TQKV_ECORRUPT);
    exit(4);
  }
}

std::vector<uint8_t> slurp(const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    perror(path);
    exit(2);
  }
  std::vector<uint8_t> d;
  uint8_t chunk[4096];
  size_t k;
  while ((k = fread(chunk, 1, sizeof chunk, f)) > 0) d.insert(d.end(), chunk, chunk + k);
  fclose(f);
  return d;
}

bool ends_with(const std::string& s, const char* tail) {
  const size_t t = strlen(tail);
  return s.size() >= t && s.compare(s.size() - t, t, tail) == 0;
}

}  // namespace

int main(int argc, char** argv) {
  long mutated_ok = 0, mutated_bad = 0;
  for (int a = 1; a < argc; ++a) {
    const std::vector<uint8_t> good = slurp(argv[a]);
    const int32_t rc = exercise(good.data(), good.size());
    if (ends_with(argv[a], ".bad")) {
      if (rc != TQKV_ECORRUPT) {
        fprintf(stderr, "%s read as valid\n", argv[a]);
        return 4;
      }
      continue;
    }
    if (rc != TQKV_OK) {
      fprintf(stderr, "%s does not read: %s\n", argv[a], tqkv_last_error());
      return 4;
    }
    // kv_disk_faults.rs: every truncation, every single-byte flip (all bits
    // and the low bit alone), one trailing byte.
    for (size_t off = 0; off < good.size(); ++off)
      expect_corrupt(std::vector<uint8_t>(good.begin(), good.begin() + off), "truncation", off);
    for (size_t at = 0; at < good.size(); ++at)
      for (uint8_t mask : {uint8_t(0xFF), uint8_t(0x01), uint8_t(0x80)}) {
        std::vector<uint8_t> bad = good;
        bad[at] ^= mask;
        expect_corrupt(bad, "byte flip", at);
      }
    {
      std::vector<uint8_t> bad = good;
      bad.push_back(0);
      expect_corrupt(bad, "trailing byte", good.size());
    }
    // Seeded mutations: overwrite, insert or delete short runs; each must
    // read or be refused, never touch memory outside its input.
    std::mt19937_64 rng(0x5eed + a);
    for (int t = 0; t < 20000; ++t) {
      std::vector<uint8_t> m = good;
      const int edits = 1 + int(rng() % 4);
      for (int e = 0; e < edits && !m.empty(); ++e) {
        const size_t at = rng() % m.size();
        const size_t len = 1 + rng() % 8;
        switch (rng() % 4) {
          case 0:
            for (size_t i = at; i < m.size() && i < at + len; ++i) m[i] = uint8_t(rng());
            break;
          case 1:
            for (size_t i = 0; i < len; ++i) m.insert(m.begin() + long(at), uint8_t(rng()));
            break;
          case 2:
            m.erase(m.begin() + long(at), m.begin() + long(std::min(m.size(), at + len)));
            break;
          default: {  // a little-endian length or count field set to an extreme
            static const uint64_t kExtreme[] = {0, 1, 0x7FFFFFFF, 0xFFFFFFFF, ~0ull, 1ull << 40};
            const uint64_t v = kExtreme[rng() % 6];
            for (size_t i = 0; i < 8 && at + i < m.size(); ++i) m[at + i] = uint8_t(v >> (8 * i));
          }
        }
      }
      const int32_t r = exercise(m.data(), m.size());
      if (r == TQKV_OK)
        ++mutated_ok;
      else if (r == TQKV_ECORRUPT)
        ++mutated_bad;
      else {
        fprintf(stderr, "mutation %d of %s: status %d\n", t, argv[a], r);
        return 4;
      }
    }
  }
  printf("lkv_sanitize: %ld inputs, mutations read %ld refused %ld\n", g_calls, mutated_ok,
         mutated_bad);
  return 0;
}
