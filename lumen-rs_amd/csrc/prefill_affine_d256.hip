// Instantiations of the affine prefill kernel for head dim 256.
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d256(int bk, int bv, bool h16) {
  return h16 ? pick_for<256, true>(bk, bv) : pick_for<256, false>(bk, bv);
}
}  // namespace prefill
}  // namespace tqkv
