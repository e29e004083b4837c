// Host-side launcher declarations shared by the C ABI and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include "nxa_common.h"

namespace nxa {

void launch_tilemap(const Params& p, int MB, int MH, int MQ, int MK, int vec16,
                    hipStream_t stream);
// Block order of each tile-map slice (MQ x MK map, slices after one another).
void launch_tile_order(const uint8_t* tilemap, int slices, int MQ, int MK, int vec16,
                       int* order, hipStream_t stream);
void launch_fwd(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_fwd16(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_delta(const Params& p, int io_dtype, hipStream_t stream);
void launch_dkdv(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_dq(const Params& p, int io_dtype, int dp, hipStream_t stream);
void launch_dkdv16(const Params& p, int io_dtype, int dp, hipStream_t stream);
// fp32 forward, dK/dV and dQ at padded head dims 64 / 128 (nxa_attn32.hip); false when
// they do not take the problem.
bool launch_fwd32(Params p, int dp, hipStream_t stream);
bool launch_dkdv32(Params p, int dp, hipStream_t stream);
bool launch_dq32(Params p, int dp, hipStream_t stream);
void launch_dq16(const Params& p, int io_dtype, int dp, hipStream_t stream);
// Padded head dim 256 (16-bit I/O), in translation units of their own.
void launch_fwd16_wide(const Params& p, int io_dtype, hipStream_t stream);
void launch_dkdv16_wide(const Params& p, int io_dtype, hipStream_t stream);
void launch_dq16_wide(const Params& p, int io_dtype, hipStream_t stream);
void launch_rms_norm(const NormParams& p, int dtype, bool bwd, hipStream_t stream);
int ssm_padded_states(int N);
int ssm_lanes_per_channel(int NP);
constexpr int kSsmChunk = 32;   // steps per chunk of the selective scan
constexpr int kSsmSub = 8;      // steps per saved sub-chunk state
constexpr int kSsmDadGroups = 16;  // row groups of the dA / dD reduction
constexpr int kSsmBlock = 256;  // channels per block of the selective scan
void launch_ssm(const SsmParams& p, bool bwd, hipStream_t stream);
// One chunk of the dbias reduction over broadcast batch / head axes.
struct DbiasReduce {
  const float* part;  // [nbh, LQ, Lk] fp32 partials of pairs bh0 .. bh0 + nbh - 1
  float* acc;         // [OB, OH, LQ, Lk] fp32 running sums
  void* out;          // dbias [OB, OH, LQ, Lk] in `dtype`, strides s (unit over Lk)
  int64_t s[3];
  int B, H, OB, OH, LQ, Lk;
  int bh0, nbh;
  int first, last;    // first chunk: sums start at zero; last: write `out`
  int dtype;
};
void launch_dbias_reduce(const DbiasReduce& r, hipStream_t stream);

}  // namespace nxa
