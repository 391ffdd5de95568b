// MFMA pre-phase instances for n = 8 streams (8 waves, KB in {1, 2, 3, 4}).
#include "mhc_pre_mfma.hpp"

namespace mhc {
hipError_t launch_pre_mfma_n8(const PreArgs& a, int kb, hipStream_t s) {
  return dispatch_pre_mode<8, 1, 2, 3, 4>(a, kb, s);
}
}  // namespace mhc
