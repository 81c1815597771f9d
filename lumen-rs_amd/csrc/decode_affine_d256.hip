// Instantiates the fused affine decode kernels for head_dim 256.
#include "decode_mfma.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d256(int bk, int bv, int G) { return pick_bits<256>(bk, bv, G); }
KernelFn pick_mfma_d256(int bk, int bv, int G, int gs, bool paged) {
  return paged ? pick_mfma<256, true>(bk, bv, G, gs) : pick_mfma<256, false>(bk, bv, G, gs);
}
}  // namespace decode
}  // namespace tqkv
