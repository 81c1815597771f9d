// Instantiates the fused affine decode kernels for head_dim 64.
#include "decode_mfma.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d64(int bk, int bv, int G) { return pick_bits<64>(bk, bv, G); }
KernelFn pick_mfma_d64(int bk, int bv, int G, int gs, bool paged) {
  return paged ? pick_mfma<64, true>(bk, bv, G, gs) : pick_mfma<64, false>(bk, bv, G, gs);
}
}  // namespace decode
}  // namespace tqkv
