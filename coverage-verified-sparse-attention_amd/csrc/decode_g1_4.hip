// Decode kernels for GQA group sizes 1-4 (decode_kernels.h): the
// launchers' explicit instantiations, one translation unit per four sizes.
#include "decode_kernels.h"

namespace cvsa {
CVSA_DECODE_INSTANTIATE(1)
CVSA_DECODE_INSTANTIATE(2)
CVSA_DECODE_INSTANTIATE(3)
CVSA_DECODE_INSTANTIATE(4)
}  // namespace cvsa
