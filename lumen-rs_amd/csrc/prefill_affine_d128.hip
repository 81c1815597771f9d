// Instantiations of the affine prefill kernel for head dim 128.
#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
KernelFn pick_d128(int bk, int bv) { return pick_for<128>(bk, bv); }
}  // namespace prefill
}  // namespace tqkv
