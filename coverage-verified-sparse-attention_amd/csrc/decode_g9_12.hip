// Decode kernels for GQA group sizes 9-12 (decode_kernels.h): the
// launchers' explicit instantiations, one translation unit per four sizes.
#include "decode_kernels.h"

namespace cvsa {
CVSA_DECODE_INSTANTIATE(9)
CVSA_DECODE_INSTANTIATE(10)
CVSA_DECODE_INSTANTIATE(11)
CVSA_DECODE_INSTANTIATE(12)
}  // namespace cvsa
