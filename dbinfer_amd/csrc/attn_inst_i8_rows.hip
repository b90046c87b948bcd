// Kernel instances of the dense int8 layout for chunk rows (matrix-core
// kernel of attn_i8_rows.hpp): 16 or 32 query vectors per workgroup, or 16
// plus a remainder tile (nvt 3).
#include "attn_i8_rows.hpp"

namespace dbi {

void* attn_instance_i8_rows(int hd, int G, int nvt) {
  switch (nvt) {
    case 1: return hd == 64 ? pick_i8_rows_g<64, 1>(G) : hd == 128 ? pick_i8_rows_g<128, 1>(G) : nullptr;
    case 2: return hd == 64 ? pick_i8_rows_g<64, 2>(G) : hd == 128 ? pick_i8_rows_g<128, 2>(G) : nullptr;
    case 3:
      return hd == 64 ? pick_i8_rows_g<64, 2, true>(G) : hd == 128 ? pick_i8_rows_g<128, 2, true>(G) : nullptr;
    default: return nullptr;
  }
}

}  // namespace dbi
