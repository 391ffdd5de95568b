// n = 8 instances of the K-streamed pre-phase kernel.
#include "mhc_pre_kstream.hpp"

namespace mhc {

hipError_t launch_pre_kstream_n8(const PreArgs& a, hipStream_t s) {
  switch (a.mode) {
    case kFull: return launch_pre_kstream_inst<8, kFull>(a, s);
    case kNoHres: return launch_pre_kstream_inst<8, kNoHres>(a, s);
    case kHead: return launch_pre_kstream_inst<8, kHead>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mhc
