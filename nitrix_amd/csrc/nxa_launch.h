// Host-side launcher declarations shared by the C ABI and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include "nxa_common.h"

namespace nxa {

void launch_tilemap(const Params& p, int MB, int MH, int MQ, int MK, int vec16,
                    hipStream_t stream);
void launch_fwd(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_fwd16(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_delta(const Params& p, int io_dtype, hipStream_t stream);
void launch_dkdv(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_dq(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_dkdv16(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_dq16(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_rms_norm(const NormParams& p, int dtype, bool bwd, hipStream_t stream);
int ssm_padded_states(int N);
int ssm_lanes_per_channel(int NP);
constexpr int kSsmChunk = 32;   // steps per chunk of the selective scan
constexpr int kSsmSub = 8;      // steps per saved sub-chunk state
constexpr int kSsmDadGroups = 16;  // row groups of the dA / dD reduction
constexpr int kSsmBlock = 256;  // channels per block of the selective scan
void launch_ssm(const SsmParams& p, bool bwd, hipStream_t stream);
void launch_dbias_reduce(const Params& p, void* out, const int64_t* out_str,
                         int OB, int OH, int LQ, hipStream_t stream);

}  // namespace nxa
