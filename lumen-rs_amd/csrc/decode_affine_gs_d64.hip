// Instantiates the MFMA decode kernels for head_dim 64 at group sizes other
// than 64 (their own unit so the builds run in parallel).
#include "decode_mfma.hpp"

namespace tqkv {
namespace decode {
KernelFn pick_mfma_gs_d64(int bk, int bv, int G, int gs) {
  switch (gs) {
    case 32: return pick_mfma_gs<64, 32>(bk, bv, G);
  }
  return nullptr;
}
}  // namespace decode
}  // namespace tqkv
