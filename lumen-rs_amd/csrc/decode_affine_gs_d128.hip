// Instantiates the MFMA decode kernels for head_dim 128 at group sizes other
// than 64 (their own unit so the builds run in parallel).
#include "decode_mfma.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_mfma_gs_d128(int bk, int bv, int G, int gs) {
  switch (gs) {
    case 32: return pick_mfma_gs<128, 32>(bk, bv, G);
    case 128: return pick_mfma_gs<128, 128>(bk, bv, G);
  }
  return nullptr;
}
}  // namespace decode
}  // namespace tqkv
