// n = 16 instances of the K-streamed pre-phase kernel.
#include "mhc_pre_kstream.hpp"

namespace mhc {

hipError_t launch_pre_kstream_n16(const PreArgs& a, hipStream_t s) { return launch_pre_kstream_mode<16>(a, s); }

}  // namespace mhc
