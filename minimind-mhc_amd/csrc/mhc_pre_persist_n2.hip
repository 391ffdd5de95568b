// Persistent MFMA pre-phase instances for n = 2 streams (KB in {1, 2, 3, 4}).
#include "mhc_pre_persist.hpp"

namespace mhc {
hipError_t launch_pre_persist_n2(const PreArgs& a, int kb, int num_cus, hipStream_t s) {
  return dispatch_persist_mode<2>(a, kb, num_cus, s);
}
}  // namespace mhc
