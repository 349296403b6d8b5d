// ptk_trace.hip — the token kernel's instances with the trace stamps of DAIZA_PTK_TRACE (per-phase
// s_memrealtime stamps of every workgroup), launched only when a trace is asked for.
#define DZ_PTK_ONLY_TU
#define DZ_PTK_TRACE
#include "ptk_kernel.h"

namespace dz {

const void* ptk_pick_trace(const PtkShape& s, bool samp) {
  if (ptk_fits(s, kPtkShape27b))
    return samp ? reinterpret_cast<const void*>(ptk_kernel_samp_trace<10, 6, 2, 1, 4, 2, 3, 12, 3, 2, 32>)
                : reinterpret_cast<const void*>(ptk_kernel_trace<10, 6, 2, 1, 4, 2, 3, 12, 3, 2, 32>);
  if (ptk_fits(s, kPtkShapeSmall))
    return samp ? reinterpret_cast<const void*>(ptk_kernel_samp_trace<1, 2, 1, 1, 1, 1, 3, 4, 1, 1, 8>)
                : reinterpret_cast<const void*>(ptk_kernel_trace<1, 2, 1, 1, 1, 1, 3, 4, 1, 1, 8>);
  return nullptr;
}

}  // namespace dz
