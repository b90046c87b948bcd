// Kernel instances of the dense int8 layout for chunk rows: 2 to 4 query
// rows per workgroup (matrix-core kernel of attn_mfma.hpp).
#include "attn_mfma.hpp"

namespace dbi {

void* attn_instance_i8_rows(int hd, int G, int cpw, int nr) {
  switch (nr) {
    case 2: return hd == 64 ? pick_i8<64, false, 2>(G, cpw) : hd == 128 ? pick_i8<128, false, 2>(G, cpw) : nullptr;
    case 3: return hd == 64 ? pick_i8<64, false, 3>(G, cpw) : hd == 128 ? pick_i8<128, false, 3>(G, cpw) : nullptr;
    case 4: return hd == 64 ? pick_i8<64, false, 4>(G, cpw) : hd == 128 ? pick_i8<128, false, 4>(G, cpw) : nullptr;
    default: return nullptr;
  }
}

}  // namespace dbi
