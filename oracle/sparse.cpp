// Page-sparse decode over an affine cache: the CPU statement the device path
// is checked against (test infrastructure only; see oracle.h).
//
// PageDigest (native_cache.rs:352-364, page_digest :407-445): elementwise
// min and max of the keys over each full 64-token page, [B, H_kv, pages, D].
// The reference digests the bf16 keys its attention reads; the keys of an
// affine cache here are its mlx::dequantize'd rows (bf16(fma(s, c, b)),
// one rounding), so min and max are exact bf16 values.
//
// sdpa_page_sparse (native_attention.rs:210-291): per (batch row, KV head),
// page p's bound is the max over the KV head's query group of
// sum_d max(q_d kmax_pd, q_d kmin_pd) (= q+ . kmax + q- . kmin); the first
// SPARSE_SINK_PAGES = 1 and last SPARSE_RECENT_PAGES = 4 full pages are
// pinned (+inf); the `keep` largest bounds are chosen, and attention runs
// over the chosen pages plus the undigested tail. With keep >= pages it is
// dense attention. keep defaults to sparse_keep_pages(pages) =
// max(pages / 8, 64) (:325-329).
//
// Two deliberate differences, both refinements where the reference leaves
// the result unspecified: the bounds are summed in f64 here (the reference
// rounds its matmul output to bf16, which creates ties), and ties are broken
// by the lower page index (the reference's argpartition leaves tied pages'
// order to the implementation). The tests check the device's choice as a
// valid top-keep under these bounds within a tolerance, and its attention
// against the oracle's over the same pages.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "oracle.h"

using namespace oracle;

extern "C" {

// key_min / key_max: [slabs, max_pages, D] bf16; pages [0, pages) of each
// slab of `cap` rows.
void oracle_page_digest_affine(const uint32_t* kw, const uint16_t* ks, const uint16_t* kb,
                               size_t slabs, size_t cap, int D, int gs, int bits, size_t pages,
                               size_t max_pages, uint16_t* key_min, uint16_t* key_max) {
  const size_t words = size_t(D) * bits / 32, groups = size_t(D / gs);
  std::vector<uint16_t> row(static_cast<size_t>(D));
  for (size_t s = 0; s < slabs; ++s)
    for (size_t p = 0; p < pages; ++p) {
      std::vector<float> mn(static_cast<size_t>(D), std::numeric_limits<float>::infinity());
      std::vector<float> mx(static_cast<size_t>(D), -std::numeric_limits<float>::infinity());
      for (size_t t = 0; t < 64; ++t) {
        const size_t r = s * cap + p * 64 + t;
        affine_dequantize_rows(kw + r * words, ks + r * groups, kb + r * groups, 1, D, gs, bits,
                               row.data());
        for (int d = 0; d < D; ++d) {
          const float v = bf16_to_f32(row[size_t(d)]);
          mn[size_t(d)] = std::min(mn[size_t(d)], v);
          mx[size_t(d)] = std::max(mx[size_t(d)], v);
        }
      }
      for (int d = 0; d < D; ++d) {
        key_min[(s * max_pages + p) * D + size_t(d)] = f32_to_bf16(mn[size_t(d)]);
        key_max[(s * max_pages + p) * D + size_t(d)] = f32_to_bf16(mx[size_t(d)]);
      }
    }
}

// bounds: [B, H_kv, pages] f64 (before pinning).
void oracle_page_bounds(const uint16_t* q, const uint16_t* key_min, const uint16_t* key_max,
                        int B, int H, int H_kv, int D, size_t pages, size_t max_pages,
                        double* bounds) {
  const int G = H / H_kv;
  for (int b = 0; b < B; ++b)
    for (int kvh = 0; kvh < H_kv; ++kvh) {
      const size_t slab = size_t(b) * H_kv + kvh;
      for (size_t p = 0; p < pages; ++p) {
        const uint16_t* mn = key_min + (slab * max_pages + p) * D;
        const uint16_t* mx = key_max + (slab * max_pages + p) * D;
        double best = -std::numeric_limits<double>::infinity();
        for (int g = 0; g < G; ++g) {
          const uint16_t* qh = q + (size_t(b) * H + size_t(kvh) * G + g) * D;
          double acc = 0.0;
          for (int d = 0; d < D; ++d) {
            const double qd = bf16_to_f32(qh[d]);
            acc += qd > 0.0 ? qd * bf16_to_f32(mx[d]) : qd * bf16_to_f32(mn[d]);
          }
          best = std::max(best, acc);
        }
        bounds[slab * pages + p] = best;
      }
    }
}

size_t oracle_sparse_keep_pages(size_t pages) { return std::max<size_t>(pages / 8, 64); }

// chosen: [units, keep] ascending page indices; keep <= pages.
void oracle_select_pages(const double* bounds, size_t units, size_t pages, size_t keep,
                         int32_t* chosen) {
  std::vector<size_t> idx(pages);
  std::vector<double> key(pages);
  for (size_t u = 0; u < units; ++u) {
    for (size_t p = 0; p < pages; ++p) {
      idx[p] = p;
      const bool pinned = p < 1 || p + 4 >= pages;
      key[p] = pinned ? std::numeric_limits<double>::infinity() : bounds[u * pages + p];
    }
    std::sort(idx.begin(), idx.end(), [&](size_t a, size_t b) {
      return key[a] != key[b] ? key[a] > key[b] : a < b;
    });
    std::vector<size_t> pick(idx.begin(), idx.begin() + long(keep));
    std::sort(pick.begin(), pick.end());
    for (size_t i = 0; i < keep; ++i) chosen[u * keep + i] = int32_t(pick[i]);
  }
}

}  // extern "C"
