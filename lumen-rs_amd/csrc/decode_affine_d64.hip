// Instantiates the fused affine decode kernels for head_dim 64.
#include "decode_affine.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d64(int bk, int bv, int G) { return pick_bits<64>(bk, bv, G); }
}  // namespace decode
}  // namespace tqkv
