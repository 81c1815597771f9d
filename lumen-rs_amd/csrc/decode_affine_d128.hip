// Instantiates the fused affine decode kernels for head_dim 128.
#include "decode_mfma.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d128(int bk, int bv, int G) { return pick_bits<128>(bk, bv, G); }
KernelFn pick_mfma_d128(int bk, int bv, int G, int gs, bool paged) {
  return paged ? pick_mfma<128, true>(bk, bv, G, gs) : pick_mfma<128, false>(bk, bv, G, gs);
}
}  // namespace decode
}  // namespace tqkv
