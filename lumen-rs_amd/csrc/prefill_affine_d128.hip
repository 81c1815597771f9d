// Instantiations of the affine prefill kernel for head dim 128.
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d128(int bk, int bv, bool h16) {
  return h16 ? pick_for<128, true>(bk, bv) : pick_for<128, false>(bk, bv);
}
}  // namespace prefill
}  // namespace tqkv
