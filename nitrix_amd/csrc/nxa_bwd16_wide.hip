// 16-bit backward kernels at padded head dim 256: dkdv256_kernel and
// dq16_kernel at one wave per SIMD.  A translation unit of its own so that
// the build can give it its own code generation flags (the machine
// scheduler's max-ILP strategy: dK/dV 7 % and dQ 6 % faster at B4 H16 L4096
// D256 than the default strategy, which is kept for head dims 64 and 128,
// where max-ILP is slower at D = 64 and no faster at D = 128).
#include "nxa_bwd16.h"

namespace nxa {

void launch_dkdv16_wide(const Params& p, int io_dtype, hipStream_t stream) {
  if (io_dtype == kF16) launch_dkdv256<f16>(p, stream);
  else launch_dkdv256<bf16>(p, stream);
}

void launch_dq16_wide(const Params& p, int io_dtype, hipStream_t stream) {
  if (io_dtype == kF16) launch_dq16_flags<f16, 256>(p, stream);
  else launch_dq16_flags<bf16, 256>(p, stream);
}

}  // namespace nxa
