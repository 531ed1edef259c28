// Packed-block protection of indexed windows, built on the GPU.
//
// Replaces the protection part of the reference's `IndexedPlan.create`
// (src/sol_attn_amd/indexed.py:27-62): for window w, query block qb and
// packed key block kb, protected = the block's keys (positions 64 kb ..
// min(64 kb + 64, len_w) - 1 of the window's sorted key list) include an
// original index inside
//   [rows[w, 64 qb] - local, rows[w, last row of qb] + local]       (local band)
// or inside any protected range [a, b).  One thread per (w, qb, kb): the
// block's keys are sorted, so "some key in [lo, hi]" is "the first key >= lo
// exists in the block and is <= hi", found by binary search over <= 64 keys.
// Blocks past a window's own keys are never protected.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr int kPlanThreads = 256;

// Position of the first of keys[begin, end) that is >= x (end if none).
__device__ __forceinline__ int64_t lower_bound(const int64_t* keys, int64_t begin, int64_t end, int64_t x) {
  while (begin < end) {
    const int64_t mid = (begin + end) >> 1;
    if (keys[mid] < x)
      begin = mid + 1;
    else
      end = mid;
  }
  return begin;
}

__device__ __forceinline__ bool touches(const int64_t* keys, int64_t begin, int64_t end, int64_t lo, int64_t hi) {
  const int64_t pos = lower_bound(keys, begin, end, lo);
  return pos < end && keys[pos] <= hi;
}

__global__ __launch_bounds__(kPlanThreads) void plan_protection_kernel(PlanParams p) {
  const int64_t i = int64_t(blockIdx.x) * kPlanThreads + threadIdx.x;
  const int64_t per_window = p.NQB * p.NKB;
  if (i >= p.W * per_window) return;
  const int64_t w = i / per_window, qb = (i % per_window) / p.NKB, kb = i % p.NKB;
  const int64_t len = p.key_lengths ? min(int64_t(p.key_lengths[w]), p.nk) : p.nk;
  const int64_t begin = kb * kBlock, end = min(begin + kBlock, len);
  bool hit = false;
  if (begin < end) {
    const int64_t* keys = p.keys + w * p.nk;
    const int64_t* rows = p.rows + w * p.nq;
    const int64_t first = rows[qb * kBlock];
    const int64_t last = rows[min(qb * kBlock + kBlock, p.nq) - 1];
    hit = touches(keys, begin, end, first - p.local, last + p.local);
    for (int r = 0; r < p.nranges && !hit; ++r)
      hit = touches(keys, begin, end, p.ranges[2 * r], p.ranges[2 * r + 1] - 1);
  }
  p.out[i] = hit ? 1 : 0;
}

}  // namespace

hipError_t launch_plan_protection(const PlanParams& p, hipStream_t stream) {
  const int64_t n = p.W * p.NQB * p.NKB;
  const unsigned blocks = unsigned((n + kPlanThreads - 1) / kPlanThreads);
  hipLaunchKernelGGL(plan_protection_kernel, dim3(blocks), dim3(kPlanThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
