// Instantiates the fused affine decode kernels for head_dim 512.
#include "decode_affine.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d512(int bk, int bv, int G) { return pick_bits<512>(bk, bv, G); }
}  // namespace decode
}  // namespace tqkv
