// Instantiations of the affine prefill kernel for head dim 512 (bf16
// operands only: the f16 variant serves shared-prefix decode up to D = 256).
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d512(int bk, int bv, bool h16) {
  return h16 ? pick_for<512, true>(bk, bv) : pick_for<512, false>(bk, bv);
}
}  // namespace prefill
}  // namespace tqkv
