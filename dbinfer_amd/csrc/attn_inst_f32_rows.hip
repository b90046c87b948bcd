// Kernel instances of the dense fp32 layout for chunk rows (matrix-core
// kernel of attn_rows.hpp): 16, 20 (a remainder tile) or 32 query vectors
// per workgroup, and the merge launch of its split records.
#include "attn_rows.hpp"

namespace dbi {

void* attn_instance_f32_rows(int hd, int G, int nvt) {
  switch (nvt) {
    case 1: return hd == 64 ? pick_rows_g<64, 1>(G) : hd == 128 ? pick_rows_g<128, 1>(G) : nullptr;
    case 2: return hd == 64 ? pick_rows_g<64, 2>(G) : hd == 128 ? pick_rows_g<128, 2>(G) : nullptr;
    case 3: return hd == 64 ? pick_rows_g<64, 3>(G) : hd == 128 ? pick_rows_g<128, 3>(G) : nullptr;
    default: return nullptr;
  }
}

void* attn_instance_f32_rows_merge(int hd, int G) {
  return hd == 64 ? pick_rows_merge_g<64>(G) : hd == 128 ? pick_rows_merge_g<128>(G) : nullptr;
}

}  // namespace dbi
