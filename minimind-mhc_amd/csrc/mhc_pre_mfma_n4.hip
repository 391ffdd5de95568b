// MFMA pre-phase instances for n = 4 streams (4 waves, KB in {2, 4, 6, 8}).
#include "mhc_pre_mfma.hpp"

namespace mhc {
hipError_t launch_pre_mfma_n4(const PreArgs& a, int kb, hipStream_t s) {
  return dispatch_pre_mode<4, 2, 4, 6, 8>(a, kb, s);
}
}  // namespace mhc
