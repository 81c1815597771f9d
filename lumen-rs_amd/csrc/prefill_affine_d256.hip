// Instantiations of the affine prefill kernel for head dim 256.
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d256(int bk, int bv) { return pick_for<256>(bk, bv); }
}  // namespace prefill
}  // namespace tqkv
