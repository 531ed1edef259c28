// Host <-> kernel parameter blocks and internal launchers (not part of the C-ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sol_device.h"

namespace sol {

// Key tokens of batch entry b: klen[b] clamped to [1, T] when per-entry
// lengths are given (ragged indexed windows), else T.  The clamp keeps every
// access inside the [B, T]-shaped index and the NKB-padded buffers whatever
// the caller's lengths hold.
__device__ __forceinline__ int batch_tokens(const int32_t* klen, int b, int T) {
  return klen ? min(max(klen[b], 1), T) : T;
}

struct PoolParams {
  TokenRows k, v;
  const int32_t* klen;  // [B] key tokens per batch entry (<= Tk), or null: all Tk
  uint16_t* ctiles;  // [B, H, NCT, 2, 64 * D] centroid tiles, or null
  uint16_t* tiles;   // [B, H, NKB, 2, 64 * D] K / V block tiles (TileLayout), or null
  float* ksum;       // [B, H, NCH, 2, D] chunk sums, null -> no moments
  float* mean;       // [B, H, D]
  float* var;        // [B, H, D]
  int B, H, Tk, NKB, NCT, NCHP;  // NCHP = 4 * NCT pooling chunks of 16 blocks
                                 // (NKB, NCT: for Tk; ragged entries use a prefix)
  int fold_in_attention;  // 1: no moments_kernel launch; the attention launch folds
                          // the chunk sums itself (AttnParams::ksum, folds_moments)
  int blocks_only;        // 1: centroid tiles only (pool_blocks_kernel; at most 16 key
                          // blocks, plain rows, no klen / tiles / ksum): the attention
                          // launch forms the moments from the tile (AttnParams::tile_moments)
};

// Key sequences whose moments the attention kernels fold from the pooling
// pass's chunk sums (AttnParams::ksum) instead of a moments_kernel launch:
// more than one 16-block chunk (one chunk's moments the pooling kernel writes
// itself) and fewer than 16 whole chunks, where moments_kernel's cascade is a
// plain sequential fold that one thread per feature repeats in a few adds.
inline bool folds_moments(int64_t nkb) { return nkb > kPoolChunk && nkb < 16 * kPoolChunk; }

// Full key covariance (covariance.hip): the full-covariance threshold
// experiment.  Partial sums over kCovSplit centroid ranges per (entry, head).
constexpr int kCovSplit = 16;

struct CovParams {
  const uint16_t* ctiles;  // [B, H, NCT, 2, 64 * D] centroid tiles (K halves read)
  const float* mean;       // [B, H, D] key centroid means
  const int32_t* klen;     // [B] key tokens per entry, or null: all Tk
  float* partial;          // [B, H, kCovSplit, D, D] workspace
  float* cov;              // [B, H, D, D]
  int B, H, Tk, NCT;
};

// Query-block pairing (pairing.hip).
constexpr int kMaxLag = 256;           // strides considered: 1 .. kMaxLag
constexpr int kMaxPairBlocks = 8192;   // query blocks per (entry, head) the lag kernel holds in LDS

struct PairParams {
  TokenRows q;
  float* qc;         // [B, H, NQB, D] FP32 query-block means (cascade order), or null
  float* means;      // [B, H, D, NQB] normalised query-block means
  float* lags;       // [B, H, D, kMaxLag] per-feature lag sums
  int32_t* strides;  // [B, H] chosen pairing stride
  int B, H, Tq, NQB;
};

struct AttnParams {
  TokenRows q;
  const int32_t* pair_stride;  // [B, H] query-block pairing stride, or null: adjacent pairs
  const int32_t* klen;         // [B] key tokens per batch entry (<= Tk), or null: all Tk
  const int64_t* out_index;    // [B, Tq] output rows of an [N, H, D] output, or null
  int64_t out_rows;            // N: rows of an out_index output (others are skipped)
  TokenRows k, v;              // key rows the kernels DMA straight into LDS (tiles null)
  const uint16_t* tiles;       // [B, H, NKB, 2, 64 * D] pooled block tiles, or null: rows of k / v
  const uint16_t* ctiles;      // [B, H, NCT, 2, 64 * D] centroid tiles
  const float* mean;           // [B, H, D]
  const float* var;            // [B, H, D]
  const float* ksum;           // [B, H, NCH, 2, D] pooling chunk sums, or null: when set (mean / var
                               // null, folds_moments(NKB), no klen) the cutoff stage folds the moments
  int tile_moments;            // 1: mean / var null, NKB <= 16, no klen: the cutoff stage forms the
                               // moments from the K centroids of centroid tile 0
  const float* cov;            // [B, H, D, D] full key covariance, or null: diagonal (var)
  const int8_t* k8;            // [B, H, NKB, 64 * D] INT8 K tiles (quantised-QK experiment), or null
  const float* k8_scale;       // [B, H, NKB] their scales
  const uint8_t* protection;   // [B, NQB, NKB] or null
  uint16_t* out;               // [B, Tq, H, D], or [N, H, D] rows out_index
  int32_t* counts;             // [B, NQB, H] or null
  uint8_t* dbg_selected;       // [B, NQB, H, NKB] or null
  float* dbg_proxy;            // [B, NQB, H, NKB] or null
  float* dbg_cutoff;           // [B, NQB, H] or null
  int B, H, Tq, Tk, NQB, NKB, NCT;  // NKB, NCT: buffer strides for Tk
  float scale, scale_log2, beta;
  int force;          // 0 finite beta, 1 beta = -inf (all exact), 2 beta = +inf
  int local_blocks;   // < 0 disables the local band
  int kv_sink_blocks, q_sink_blocks;
  int workgroup_form;  // 0: by launch size; 1 / 2: query blocks per workgroup of
                       // sol_attention_kernel
  int splits;          // key-range parts per front (query-sink) tile, >= 1 (sol_task)
  float* partial;      // their partial states when splits > 1: rows [B H][front][G 64][D + 4]
  uint32_t* mask;      // [B, H, NQB, NW] routing decisions (route_kernel), bit j of word w = key block 32 w + j;
                       // null: the attention kernel routes tile by tile
  int NW;              // ceil(NKB / 32)
  const float* qc;     // [B, H, NQB, D] FP32 query-block means for route_kernel, or null (formed from Q)
  int32_t* order;      // [B H, NQB] with mask: the regular query tiles of a two-block launch in
                       // the order order_kernel deals them to the XCDs, or null: tile order
};

// Indexed-window protection (plan.hip).
struct PlanParams {
  const int64_t* rows;         // [W, nq] sorted original query rows
  const int64_t* keys;         // [W, nk] sorted original key indices
  const int32_t* key_lengths;  // [W] keys per window (clamped to nk), or null: nk
  const int64_t* ranges;       // [nranges, 2] protected ranges [a, b)
  uint8_t* out;                // [W, NQB, NKB]
  int64_t W, nq, nk, NQB, NKB, local;
  int nranges;
};

// INT8 K tiles of the quantised-QK experiment (quant.hip).
struct QuantParams {
  TokenRows k;
  const int32_t* klen;  // [B] key tokens per batch entry (<= Tk), or null: all Tk
  int8_t* k8;           // [B, H, NKB, 64 * D]
  float* scale;         // [B, H, NKB]
  int B, H, Tk, NKB;
  int shifted;          // partial last blocks as the rows-mode attention tiles hold them
};

// Key-split groups of sol_small_kernel for a launch of `blocks` query blocks
// (over all entries and heads) against nkb key blocks, or 0 when the launch
// takes sol_attention_kernel.  Small launches (at most kSmallBlocks query
// blocks, a workgroup each) leave most SIMDs idle, so their time is one
// workgroup's tile chain: KS groups of two waves split it KS ways, within the
// LDS of two ring slots per group (4 groups at D = 64, 2 at D = 128), while
// the chain stays at most kSmallChain steps.  Longer key sequences go to the
// one-block kernel, whose query-sink tiles split over workgroups instead.
constexpr int64_t kSmallBlocks = 256;
constexpr int64_t kSmallChain = 16;
inline int small_key_split(int64_t blocks, int64_t nkb, int64_t head_dim) {
  const int ks = head_dim == 64 ? 4 : 2;
  return blocks <= kSmallBlocks && nkb <= kSmallChain * ks ? ks : 0;
}

hipError_t launch_pool(const PoolParams& p, int D, hipStream_t stream);
hipError_t launch_quantize_keys(const QuantParams& p, int D, hipStream_t stream);
hipError_t launch_route(const AttnParams& p, int D, hipStream_t stream);
hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream);
hipError_t launch_dense(const AttnParams& p, int D, hipStream_t stream);
hipError_t launch_pairing(const PairParams& p, int D, hipStream_t stream);
hipError_t launch_plan_protection(const PlanParams& p, hipStream_t stream);
hipError_t launch_covariance(const CovParams& p, int D, hipStream_t stream);

}  // namespace sol
