// C-ABI shim over the reference's own header-only unpack
// (src/loader/w4a16_unpack.h, compiled from where it lies under the reference
// tree by oracle/Makefile). Test infrastructure: it cross-checks the oracle's
// restatement of that header; nothing in the product links it.
#include <cstdint>
#include "w4a16_unpack.h"

extern "C" {
int32_t ref_w4_q(const uint32_t* packed, int64_t in_features, int64_t o, int64_t i) {
  return qwen::w4_q(packed, in_features, o, i);
}
int32_t ref_w4_zp(const uint32_t* zp, int64_t num_groups, int64_t o, int64_t g) {
  return qwen::w4_zp(zp, num_groups, o, g);
}
int32_t ref_unpack_nibble(const uint32_t* words, int64_t e) { return qwen::unpack_nibble(words, e); }
}
