// 16-bit forward kernel at padded head dim 256 (one wave per SIMD).  A
// translation unit of its own so that the build can give it its own code
// generation flags (MFMA operands and results forced into VGPRs: 11 %
// faster at B4 H16 L4096 D256 than the compiler's default choice).
#include "nxa_fwd16.h"

namespace nxa {

void launch_fwd16_wide(const Params& p, int io_dtype, hipStream_t stream) {
  if (io_dtype == kF16) launch_fwd16_flags<f16, 256>(p, stream);
  else launch_fwd16_flags<bf16, 256>(p, stream);
}

}  // namespace nxa
