// INT8 K tiles for the quantised-QK experiment of the reference's roadmap
// (ROADMAP.md:14-16: "separately measured INT8 QK ... Preserve a BF16
// control"), which the reference does not implement.
//
// Per key block (64 keys x D): one symmetric scale s_k = max|K| / 127 over
// the block's keys, K8 = rint(K * (127 / max|K|)) clamped to +-127 (0 for an
// all-zero block), stored in the bank-swizzled K8Layout the attention
// kernel's INT8 products read, with the block's rows where the attention
// kernels' BF16 V tile has them: rows 64 j .. of the sequence, zero past its
// end, or -- for the partial last block of a sequence whose V rows the
// attention kernel reads shifted back (p.shifted) -- the sequence's last 64
// rows, of which only the block's own keys (the last len) set the scale.
// HBM-bound: D * 128 bytes read and D * 64 + 4 written per block.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr int kQuantThreads = 256;

template <int D>
__global__ __launch_bounds__(kQuantThreads) void quantize_keys_kernel(QuantParams p) {
  constexpr int kChunks = kBlock * D / 16;  // INT8 chunks (16 features) per block
  constexpr int kPer = kChunks / kQuantThreads;
  constexpr int kRowChunks = D / 16;
  static_assert(kPer * kQuantThreads == kChunks, "chunks split evenly over the workgroup");
  __shared__ float s_max[kQuantThreads / kWave];

  const int j = blockIdx.x % p.NKB;
  const int bh = blockIdx.x / p.NKB;
  const int h = bh % p.H, b = bh / p.H;
  const int tk = batch_tokens(p.klen, b, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  if (j >= nkb) return;  // past this entry's blocks (uniform per workgroup)
  const int len = min(kBlock, tk - kBlock * j);
  const bool shifted = p.shifted && len < kBlock;
  const int row0 = shifted ? tk - kBlock : kBlock * j;  // sequence row of tile row 0
  const int first = shifted ? kBlock - len : 0;          // tile rows first .. first + len - 1 are the block's
  int8_t* dst = p.k8 + int64_t(blockIdx.x) * K8Layout<D>::kBytes;
  const int tid = threadIdx.x, lane = tid & 63;

  u32x4 raw[kPer][2];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kQuantThreads * i;
    const int row = c / kRowChunks, ch = c % kRowChunks;
    const bool present = row >= first && row < first + len;
    const bool readable = shifted || present;  // shifted rows all exist
    const uint16_t* src = p.k.row(b, row0 + (readable ? row : first), h) + 16 * ch;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      raw[i][hf] = readable ? load16(src + 8 * hf) : zero_u32x4();
      if (present) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = raw[i][hf][e >> 1];
          amax = fmaxf(amax, fabsf(bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu))));
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if (lane == 0) s_max[tid >> 6] = amax;
  __syncthreads();
  amax = s_max[0];
#pragma unroll
  for (int w = 1; w < kQuantThreads / kWave; ++w) amax = fmaxf(amax, s_max[w]);
  const float inv = amax > 0.f ? __fdiv_rn(127.f, amax) : 0.f;

#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = tid + kQuantThreads * i;
    const int row = c / kRowChunks, ch = c % kRowChunks;
    u32x4 out;
#pragma unroll
    for (int wd = 0; wd < 4; ++wd) {
      uint32_t packed = 0;
#pragma unroll
      for (int bt = 0; bt < 4; ++bt) {
        const int e = 4 * wd + bt;  // feature 16 ch + e
        const uint32_t w = raw[i][e >> 3][(e & 7) >> 1];
        const float x = bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu));
        const int q = int(fminf(fmaxf(rintf(__fmul_rn(x, inv)), -127.f), 127.f));
        packed |= (uint32_t(q) & 0xFFu) << (8 * bt);
      }
      out[wd] = packed;
    }
    *reinterpret_cast<u32x4*>(dst + K8Layout<D>::offset(row, ch)) = out;
  }
  if (tid == 0) p.scale[blockIdx.x] = __fdiv_rn(amax, 127.f);
}

}  // namespace

hipError_t launch_quantize_keys(const QuantParams& p, int D, hipStream_t stream) {
  const dim3 grid(unsigned(int64_t(p.B) * p.H * p.NKB));
  if (D == 128)
    hipLaunchKernelGGL(quantize_keys_kernel<128>, grid, dim3(kQuantThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(quantize_keys_kernel<64>, grid, dim3(kQuantThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
