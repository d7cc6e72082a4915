// MoE FFN over MLX affine experts of 2 and 3 bits: the instantiations of moe_ffn_affine for those
// widths (see moe.hip), in a translation unit of their own so that they compile in parallel with
// the rest of the library.
#define ISHZ_MOE_BODY_ONLY
#include "moe.hip"

namespace ishz {

int moe_affine_w23(int bits, int group, bool bf16s, ISHZ_MOE_AFFINE_ARGS) {
#define ISHZ_MA(B, G)                                                                        \
  return bf16s ? moe_ffn_affine<FAffineN<B, G, true>>(ISHZ_MOE_AFFINE_PASS)                  \
               : moe_ffn_affine<FAffineN<B, G, false>>(ISHZ_MOE_AFFINE_PASS)
  switch (bits) {
    case 2:
      if (group == 64) ISHZ_MA(2, 64);
      ISHZ_MA(2, 128);
    case 3:
      if (group == 64) ISHZ_MA(3, 64);
      ISHZ_MA(3, 128);
  }
#undef ISHZ_MA
  return decline("affine experts of 2 to 8 bits are decoded in-kernel");
}

}  // namespace ishz
