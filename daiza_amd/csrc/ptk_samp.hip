// ptk_samp.hip — the sampled instances of the persistent token kernel (ptk_kernel_samp: the token
// kernel with the draws of dz_decode_sample inside it), in a code object of their own.
#define DZ_PTK_ONLY_TU
#include "ptk_kernel.h"

namespace dz {

const void* ptk_pick_samp(const PtkShape& s) {
  if (ptk_fits(s, kPtkShape27b))
    return reinterpret_cast<const void*>(ptk_kernel_samp<10, 6, 2, 1, 4, 2, 3, 12, 3, 2, 32>);
  if (ptk_fits(s, kPtkShapeSmall))
    return reinterpret_cast<const void*>(ptk_kernel_samp<1, 2, 1, 1, 1, 1, 3, 4, 1, 1, 8>);
  return nullptr;
}

}  // namespace dz
