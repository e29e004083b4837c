// 16-bit forward kernels at padded head dims 64 and 128, and the dispatch
// over head dims (256 lives in nxa_fwd16_wide.hip).
#include "nxa_fwd16.h"

namespace nxa {

void launch_fwd16(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (dp == 256) {
    launch_fwd16_wide(p, io_dtype, stream);
  } else if (io_dtype == kF16) {
    if (dp == 64) launch_fwd16_flags<f16, 64>(p, stream);
    else launch_fwd16_flags<f16, 128>(p, stream);
  } else {
    if (dp == 64) launch_fwd16_flags<bf16, 64>(p, stream);
    else launch_fwd16_flags<bf16, 128>(p, stream);
  }
}

}  // namespace nxa
