// Instances of attn_kernel for the f32 dense layout, raw-projection producer.
#include "attn_kernel.hpp"

namespace dbi {

void* attn_instance_0_1(int hd, int G, int cpw) {
  return hd == 64 ? pick_g<64, 0, true>(G, cpw)
       : hd == 128 ? pick_g<128, 0, true>(G, cpw)
                   : nullptr;
}

}  // namespace dbi
