// Full key covariance per (batch entry, head), for the full-covariance
// threshold experiment (roadmap item 4 of the reference, ROADMAP.md:14-16;
// the reference implements only the diagonal of `_moments`,
// src/sol_attn_amd/kernels.py:30-49):
//   cov = mean_j Kc_j Kc_j^T - mu mu^T
// over the entry's BF16 block centroids Kc_j (population, unweighted by
// ragged length, as the diagonal estimator), with mu the diagonal pass's
// mean.  Two launches: kCovSplit workgroups per (entry, head) each sum the
// outer products of one range of centroids (thread (di, ei) owns the 8 x 8
// tile of rows 8 di.. and columns 8 ei..), then one workgroup per (entry,
// head) folds the ranges in order and subtracts mu mu^T.  FP32 throughout.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr int kCovThreads = 256;

__device__ __forceinline__ void unpack8(u32x4 x, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = x[e >> 1];
    f[e] = bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu));
  }
}

template <int D>
__global__ __launch_bounds__(kCovThreads) void covariance_partial_kernel(CovParams p) {
  using TL = TileLayout<D>;
  constexpr int DC = D / 8;  // 8-feature chunks: threads (di, ei) for di, ei < DC
  const int bh = blockIdx.x, split = blockIdx.y;
  const int tk = batch_tokens(p.klen, bh / p.H, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  const int per = (nkb + kCovSplit - 1) / kCovSplit;
  const int j0 = min(nkb, split * per), j1 = min(nkb, j0 + per);
  const int t = threadIdx.x;
  if (t >= DC * DC) return;
  const int di = t / DC, ei = t % DC;
  float acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[i][k] = 0.f;
  const uint16_t* ctiles = p.ctiles + int64_t(bh) * p.NCT * 2 * TL::kElems;
  for (int j = j0; j < j1; ++j) {
    const uint16_t* tile = ctiles + int64_t(j / kBlock) * 2 * TL::kElems;  // its K half
    float x[8], y[8];
    unpack8(load16(tile + TL::k_offset(j % kBlock, di)), x);
    unpack8(load16(tile + TL::k_offset(j % kBlock, ei)), y);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[i][k] = fmaf(x[i], y[k], acc[i][k]);
  }
  float* out = p.partial + (int64_t(bh) * kCovSplit + split) * D * D;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) out[(8 * di + i) * D + 8 * ei + k] = acc[i][k];
}

template <int D>
__global__ __launch_bounds__(kCovThreads) void covariance_finish_kernel(CovParams p) {
  const int bh = blockIdx.x;
  const int tk = batch_tokens(p.klen, bh / p.H, p.Tk);
  const float n = float((tk + kBlock - 1) / kBlock);
  const float* part = p.partial + int64_t(bh) * kCovSplit * D * D;
  const float* mu = p.mean + int64_t(bh) * D;
  for (int idx = threadIdx.x; idx < D * D; idx += kCovThreads) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < kCovSplit; ++r) s += part[int64_t(r) * D * D + idx];
    p.cov[int64_t(bh) * D * D + idx] = s / n - mu[idx / D] * mu[idx % D];
  }
}

}  // namespace

hipError_t launch_covariance(const CovParams& p, int D, hipStream_t stream) {
  const dim3 grid(unsigned(p.B) * p.H, kCovSplit);
  if (D == 128) {
    hipLaunchKernelGGL(covariance_partial_kernel<128>, grid, dim3(kCovThreads), 0, stream, p);
    hipLaunchKernelGGL(covariance_finish_kernel<128>, dim3(p.B * p.H), dim3(kCovThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL(covariance_partial_kernel<64>, grid, dim3(kCovThreads), 0, stream, p);
    hipLaunchKernelGGL(covariance_finish_kernel<64>, dim3(p.B * p.H), dim3(kCovThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace sol
