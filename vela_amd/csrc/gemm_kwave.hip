// Instantiations of the K-split-over-waves kernel (kwave_kernel.h): sources I16, I8 and CONV16,
// epilogues PLAIN, SPLIT3, GEGLU and GELU.
#include "kwave_kernel.h"

namespace vk {

template <int SRC>
static hipError_t launch_kwave_src(int epi, const GemmParams& p, hipStream_t st) {
    switch (epi) {
    case EPI_PLAIN: return launch_kwave_t<SRC, EPI_PLAIN>(p, st);
    case EPI_SPLIT3: return launch_kwave_t<SRC, EPI_SPLIT3>(p, st);
    case EPI_GEGLU: return launch_kwave_t<SRC, EPI_GEGLU>(p, st);
    case EPI_GELU: return launch_kwave_t<SRC, EPI_GELU>(p, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_kwave(int src, int epi, const GemmParams& p, hipStream_t st) {
    switch (src) {
    case SRC_I16: return launch_kwave_src<SRC_I16>(epi, p, st);
    case SRC_I8: return launch_kwave_src<SRC_I8>(epi, p, st);
    case SRC_CONV16: return launch_kwave_src<SRC_CONV16>(epi, p, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace vk
