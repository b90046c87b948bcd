// Kernel instances of the dense int8 layout, plain inputs, one query row per
// workgroup (matrix-core kernel of attn_mfma.hpp).
#include "attn_mfma.hpp"

namespace dbi {

void* attn_instance_1_0(int hd, int G, int cpw) {
  return hd == 64 ? pick_i8<64, false, 1>(G, cpw) : hd == 128 ? pick_i8<128, false, 1>(G, cpw) : nullptr;
}

}  // namespace dbi
