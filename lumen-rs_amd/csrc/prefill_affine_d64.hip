// Instantiations of the affine prefill kernel for head dim 64.
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d64(int bk, int bv) { return pick_for<64>(bk, bv); }
}  // namespace prefill
}  // namespace tqkv
