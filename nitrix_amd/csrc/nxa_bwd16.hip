// 16-bit backward kernels at padded head dims 64 and 128, and the dispatch
// over head dims (256 lives in nxa_bwd16_wide.hip).
#include "nxa_bwd16.h"

namespace nxa {

template <typename T>
static void launch_dkdv16_dp(const Params& p, int dp, hipStream_t stream) {
  if (dp == 64) {
    if (p.causal) launch_dkdv16_db<T, 64, true>(p, stream);
    else launch_dkdv16_db<T, 64, false>(p, stream);
  } else {
    if (p.causal) launch_dkdv16_db<T, 128, true>(p, stream);
    else launch_dkdv16_db<T, 128, false>(p, stream);
  }
}

void launch_dkdv16(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (dp == 256) launch_dkdv16_wide(p, io_dtype, stream);
  else if (io_dtype == kF16) launch_dkdv16_dp<f16>(p, dp, stream);
  else launch_dkdv16_dp<bf16>(p, dp, stream);
}

template <typename T>
static void launch_dq16_dp(const Params& p, int dp, hipStream_t stream) {
  if (dp == 64) launch_dq16_flags<T, 64>(p, stream);
  else launch_dq16_flags<T, 128>(p, stream);
}

void launch_dq16(const Params& p, int io_dtype, int dp, hipStream_t stream) {
  if (dp == 256) launch_dq16_wide(p, io_dtype, stream);
  else if (io_dtype == kF16) launch_dq16_dp<f16>(p, dp, stream);
  else launch_dq16_dp<bf16>(p, dp, stream);
}

}  // namespace nxa
