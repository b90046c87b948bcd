// Instances of attn_kernel for the i8 ring layout, raw-projection producer.
#include "attn_kernel.hpp"

namespace dbi {

void* attn_instance_3_1(int hd, int G, int cpw) {
  return hd == 64 ? pick_g<64, 3, true>(G, cpw)
       : hd == 128 ? pick_g<128, 3, true>(G, cpw)
                   : nullptr;
}

}  // namespace dbi
