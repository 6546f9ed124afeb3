// Decode kernels for GQA group sizes 13-16 (decode_kernels.h): the
// launchers' explicit instantiations, one translation unit per four sizes.
#include "decode_kernels.h"

namespace cvsa {
CVSA_DECODE_INSTANTIATE(13)
CVSA_DECODE_INSTANTIATE(14)
CVSA_DECODE_INSTANTIATE(15)
CVSA_DECODE_INSTANTIATE(16)
}  // namespace cvsa
