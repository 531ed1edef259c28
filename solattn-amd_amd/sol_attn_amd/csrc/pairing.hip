// Query-block pairing for the SOL attention workgroups.
//
// A SOL workgroup holds two query blocks and streams the union of their
// selected key blocks, so its time follows the union while its useful work
// follows the sum: pairing query blocks whose selections overlap shortens the
// stream.  A query block's selection is a function of its mean (the routing
// proxy is q_mean . k_mean, tested against a cutoff built from the same
// q_mean), so the pairing is chosen from the query-block means before any
// routing, per (batch entry, head):
//   1. m_i = mean of query block i, normalised to unit length;
//   2. c(s) = mean over i of m_i . m_{i+s} for every lag s = 1 .. kMaxLag;
//   3. the stride s maximising the mean cosine of the pairs the attention
//      kernel would form at that stride -- (i, i+s) inside each full run of
//      2 s blocks, adjacent pairs after the last full run:
//        score(s) = (covered(s) c(s) + (NQB - covered(s)) c(1)) / NQB.
// Lag s = 1 is the adjacent pairing.  For a video latent laid out frame by
// frame with W blocks per frame this finds s = W (the same spatial block in
// the next frame).  Pairing changes which blocks share a workgroup, never a
// block's own computation: outputs are identical for every stride.
// The reference runs one Triton program per query block and has no
// counterpart.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr int kMeanThreads = 256;  // four waves
constexpr int kMeanChunk = 16;     // query blocks per workgroup

// Query-block means: with p.qc, the FP32 means themselves, qc[((b H + h) NQB
// + i) D + d] (the routing kernel's Qc); and the normalised means,
// m[((b H + h) D + d) NQB + i] (lag-major rows
// so that the lag kernel reads one feature of one head contiguously).  One
// workgroup per (batch entry, head, 16 consecutive query blocks), in the
// pooling kernel's load shape: each lane holds 16 rows x 16 bytes of one
// block in flight (non-temporal: Q is read once here), the four waves take
// the chunk's blocks in turn, and the lane quarters' partial sums are folded
// with shuffles.  Each block mean is normalised by its norm over D, staged in
// LDS, and written out as runs of consecutive blocks per feature.  Heads vary
// fastest over the grid, so the workgroups in flight read whole token rows.
template <int D>
__global__ __launch_bounds__(kMeanThreads) void qblock_means_kernel(PairParams p) {
  constexpr int DC = D / 8;          // 16-byte chunks per row
  constexpr int LPB = DC * 4;        // lanes per block: 4 quarters of 16 rows
  constexpr int BPI = kWave / LPB;   // blocks per wave iteration
  constexpr int NW = kMeanThreads / kWave;
  constexpr int ITERS = kMeanChunk / (NW * BPI);
  static_assert(ITERS * NW * BPI == kMeanChunk, "a workgroup covers one chunk");
  __shared__ float m[kMeanChunk][D + 1];  // padded: the write-out reads columns
  const int c = blockIdx.x / (p.B * p.H);
  const int bh = blockIdx.x % (p.B * p.H);
  const int h = bh % p.H, b = bh / p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane / LPB, r4 = (lane % LPB) / DC, dc = lane % DC;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int jb = (wave * ITERS + it) * BPI + sub;  // block inside this chunk
    const int i = c * kMeanChunk + jb;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int qlen = 0;
    if (i < p.NQB) {
      qlen = min(kBlock, p.Tq - kBlock * i);
      u32x4 x[16];
      load_rows16<16, true>(p.q, b, kBlock * i + 16 * r4, kBlock * i + qlen - 1, h, 8 * dc, x);
#pragma unroll
      for (int r = 0; r < 16; ++r)  // rows past the block are zero
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = x[r][e >> 1];
          s[e] = __fadd_rn(s[e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)));
        }
    }
    // The four 16-row quarter sums fold in order, ((q0 + q1) + q2) + q3:
    // torch's cascade order for a 64-row block, so the FP32 mean equals the
    // reference oracle's `_means` (reference.py:13-15) bit for bit.
    float n2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c1 = __shfl(s[e], lane + DC), c2 = __shfl(s[e], lane + 2 * DC), c3 = __shfl(s[e], lane + 3 * DC);
      s[e] = qlen > 0 ? __fdiv_rn(__fadd_rn(__fadd_rn(__fadd_rn(s[e], c1), c2), c3), float(qlen)) : 0.f;
      n2 += s[e] * s[e];
    }
    if (p.qc && r4 == 0 && i < p.NQB) {
      float* dst = p.qc + (int64_t(bh) * p.NQB + i) * D + 8 * dc;
      *reinterpret_cast<f32x4*>(dst) = f32x4{s[0], s[1], s[2], s[3]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{s[4], s[5], s[6], s[7]};
    }
    // The DC lanes of quarter 0 of a block are consecutive and DC-aligned.
#pragma unroll
    for (int off = 1; off < DC; off <<= 1) n2 += __shfl_xor(n2, off);
    const float inv = n2 > 0.f ? rsqrtf(n2) : 0.f;
    if (r4 == 0)
#pragma unroll
      for (int e = 0; e < 8; ++e) m[jb][8 * dc + e] = s[e] * inv;
  }
  __syncthreads();
  constexpr int F = kMeanChunk * D / kMeanThreads;  // blocks per thread in the write-out
  const int d = tid / (kMeanChunk / F), j0 = (tid % (kMeanChunk / F)) * F;
  float* dst = p.means + (int64_t(bh) * D + d) * p.NQB + c * kMeanChunk;
#pragma unroll
  for (int j = j0; j < j0 + F; ++j)
    if (c * kMeanChunk + j < p.NQB) dst[j] = m[j][d];
}

// Lag sums of one feature d of one (batch entry, head): thread t holds the
// four lags s = 4 t + 1 .. 4 t + 4, sum over i of m_i[d] m_{i+s}[d], each
// in ascending i.  Steps go four at a time: a step block needs m_i .. m_{i+3}
// (the same for every lane) and the lane's window m_{i+s0} .. m_{i+s0+7}, of
// which the first four came with the previous block, and the reads for the
// next block are issued before this block's products, so their latency
// overlaps them.  The LDS copy is zero-padded past NQB (kLagPad values, enough
// for the block after the last), so terms past the end add exact zeros.
// Value k sits at word lag_word(k) = k + k / 32: the lanes' window reads lie
// 4 values apart, and without the pad word after every 32 values groups of 8
// lanes would hit the same bank; with it the lanes 8 apart fall in
// neighbouring banks.
constexpr int kLagThreads = kMaxLag / 4;
constexpr int kLagPad = kMaxLag + 16;

__host__ __device__ constexpr int lag_word(int k) { return k + (k >> 5); }

__global__ __launch_bounds__(kLagThreads) void pair_lag_kernel(PairParams p, int D) {
  extern __shared__ float x[];  // lag_word(NQB + kLagPad - 1) + 1 floats
  const int d = blockIdx.x, bh = blockIdx.y, n = p.NQB;
  const float* src = p.means + (int64_t(bh) * D + d) * n;
  for (int i = threadIdx.x; i < n + kLagPad; i += kLagThreads) x[lag_word(i)] = i < n ? src[i] : 0.f;
  __syncthreads();
  const int s0 = 4 * threadIdx.x + 1;
  float v[8], xc[4];  // v: m_{i+s0} .. m_{i+s0+7}; xc: m_i .. m_{i+3}
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = x[lag_word(s0 + u)];
#pragma unroll
  for (int u = 0; u < 4; ++u) xc[u] = x[lag_word(u)];
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < n; i += 4) {
    float xn[4], wn[4];  // the next block's m_{i+4} .. m_{i+7} and m_{i+s0+8} .. m_{i+s0+11}
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      xn[u] = x[lag_word(i + 4 + u)];
      wn[u] = x[lag_word(i + s0 + 8 + u)];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) a[k] = fmaf(xc[u], v[u + k], a[k]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      xc[u] = xn[u];
      v[u] = v[u + 4];
      v[u + 4] = wn[u];
    }
  }
  float* dst = p.lags + (int64_t(bh) * D + d) * kMaxLag + 4 * threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) dst[k] = a[k];
}

// Per (batch entry, head): mean cosine per lag, pairing score per stride,
// argmax (the smallest stride on ties).
__global__ __launch_bounds__(kMaxLag) void pair_pick_kernel(PairParams p, int D) {
  __shared__ float s_score[kMaxLag];
  __shared__ float s_c1;
  const int bh = blockIdx.x, t = threadIdx.x, s = t + 1;
  const int n = p.NQB;
  float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // loads in flight
  for (int d = 0; d < D; d += 8)
#pragma unroll
    for (int u = 0; u < 8; ++u) part[u] += p.lags[(int64_t(bh) * D + d + u) * kMaxLag + t];
  const float r = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
  const float c = n - s > 0 ? r / float(n - s) : 0.f;  // mean cosine at lag s
  if (t == 0) s_c1 = c;
  __syncthreads();
  const int covered = (n / (2 * s)) * (2 * s);  // blocks that a stride-s pairing pairs at lag s
  s_score[t] = covered > 0 ? (float(covered) * c + float(n - covered) * s_c1) / float(n) : -2.f;
  __syncthreads();
  if (t == 0) {
    int best = 0;
    for (int i = 1; i < kMaxLag; ++i)
      if (s_score[i] > s_score[best]) best = i;
    p.strides[bh] = best + 1;
  }
}

}  // namespace

hipError_t launch_pairing(const PairParams& p, int D, hipStream_t stream) {
  const unsigned mean_grid = unsigned((p.NQB + kMeanChunk - 1) / kMeanChunk) * unsigned(p.B * p.H);
  if (D == 128)
    hipLaunchKernelGGL(qblock_means_kernel<128>, dim3(mean_grid), dim3(kMeanThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(qblock_means_kernel<64>, dim3(mean_grid), dim3(kMeanThreads), 0, stream, p);
  hipLaunchKernelGGL(pair_lag_kernel, dim3(D, p.B * p.H), dim3(kLagThreads),
                     (lag_word(p.NQB + kLagPad - 1) + 1) * sizeof(float), stream, p, D);
  hipLaunchKernelGGL(pair_pick_kernel, dim3(p.B * p.H), dim3(kMaxLag), 0, stream, p, D);
  return hipGetLastError();
}

}  // namespace sol
