// Instances of attn_kernel for the i8 dense layout.
#include "attn_kernel.hpp"

namespace dbi {

void* attn_instance_1_0(int hd, int G, int cpw) {
  return hd == 64 ? pick_g<64, 1, false>(G, cpw)
       : hd == 128 ? pick_g<128, 1, false>(G, cpw)
                   : nullptr;
}

}  // namespace dbi
