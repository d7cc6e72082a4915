// MoE FFN over MLX affine experts of 5, 6 and 7 bits: the instantiations of moe_ffn_affine for those
// widths (see moe.hip), in a translation unit of their own so that they compile in parallel with
// the rest of the library.
#define ISHZ_MOE_BODY_ONLY
#include "moe.hip"

namespace ishz {

int moe_affine_w567(int bits, int group, bool bf16s, ISHZ_MOE_AFFINE_ARGS) {
#define ISHZ_MA(B, G)                                                                        \
  return bf16s ? moe_ffn_affine<FAffineN<B, G, true>>(ISHZ_MOE_AFFINE_PASS)                  \
               : moe_ffn_affine<FAffineN<B, G, false>>(ISHZ_MOE_AFFINE_PASS)
  switch (bits) {
    case 5:
      if (group == 64) ISHZ_MA(5, 64);
      ISHZ_MA(5, 128);
    case 6:
      if (group == 64) ISHZ_MA(6, 64);
      ISHZ_MA(6, 128);
    case 7:
      if (group == 64) ISHZ_MA(7, 64);
      ISHZ_MA(7, 128);
  }
#undef ISHZ_MA
  return decline("affine experts of 2 to 8 bits are decoded in-kernel");
}

}  // namespace ishz
