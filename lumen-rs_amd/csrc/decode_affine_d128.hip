// Instantiates the fused affine decode kernels for head_dim 128.
#include "decode_affine.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_d128(int bk, int bv, int G) { return pick_bits<128>(bk, bv, G); }
}  // namespace decode
}  // namespace tqkv
