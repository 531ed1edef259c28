// Host <-> kernel parameter blocks and internal launchers (not part of the C-ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sol_device.h"

namespace sol {

struct PoolParams {
  TokenRows k, v;
  uint16_t* kc;     // [B, H, NKB, D] or null (no centroids)
  uint16_t* vct;    // [B, H, D, NKBP] or null
  uint16_t* tiles;  // [B, H, NKB, 2, 64 * D] swizzled K / V^T block tiles, or null
  float* ksum;      // [B, H, NCH, 2, D] chunk sums, null -> no moments
  float* mean;      // [B, H, D]
  float* var;       // [B, H, D]
  int B, H, Tk, NKB, NKBP, NCHP;
};

struct AttnParams {
  TokenRows q;
  const uint16_t* tiles;       // [B, H, NKB, 2, 64 * D] from the pooling pass
  const uint16_t* kc;          // [B, H, NKB, D]
  const uint16_t* vct;         // [B, H, D, NKBP]
  const float* mean;           // [B, H, D]
  const float* var;            // [B, H, D]
  const uint8_t* protection;   // [B, NQB, NKB] or null
  uint16_t* out;               // [B, Tq, H, D]
  int32_t* counts;             // [B, NQB, H] or null
  uint8_t* dbg_selected;       // [B, NQB, H, NKB] or null
  float* dbg_proxy;            // [B, NQB, H, NKB] or null
  float* dbg_cutoff;           // [B, NQB, H] or null
  int B, H, Tq, Tk, NQB, NKB, NKBP;
  float scale, scale_log2, beta;
  int force;          // 0 finite beta, 1 beta = -inf (all exact), 2 beta = +inf
  int local_blocks;   // < 0 disables the local band
  int kv_sink_blocks, q_sink_blocks;
};

hipError_t launch_pool(const PoolParams& p, int D, hipStream_t stream);
hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream);
hipError_t launch_dense(const AttnParams& p, int D, hipStream_t stream);

}  // namespace sol
