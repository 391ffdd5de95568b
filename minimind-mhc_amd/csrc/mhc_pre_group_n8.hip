// Small-batch MFMA pre-phase instances for n = 8 streams (KB in {1, 2, 3, 4}).
#include "mhc_pre_group.hpp"

namespace mhc {
hipError_t launch_pre_group_n8(const PreArgs& a, int num_cus, hipStream_t s) {
  return dispatch_group_mode<8>(a, num_cus, s);
}
}  // namespace mhc
