// Decode kernels for GQA group sizes 5-8 (decode_kernels.h): the
// launchers' explicit instantiations, one translation unit per four sizes.
#include "decode_kernels.h"

namespace cvsa {
CVSA_DECODE_INSTANTIATE(5)
CVSA_DECODE_INSTANTIATE(6)
CVSA_DECODE_INSTANTIATE(7)
CVSA_DECODE_INSTANTIATE(8)
}  // namespace cvsa
