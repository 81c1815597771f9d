// Instantiates the fused affine decode kernels for head_dim 256.
#include "decode_affine.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d256(int bk, int bv, int G) { return pick_bits<256>(bk, bv, G); }
}  // namespace decode
}  // namespace tqkv
