// K/V block pooling and diagonal key moments for SOL routed attention.
//
// Replaces the reference's `_pool` + `_pooled` (src/sol_attn_amd/kernels.py:16-27,
// 185-190) and `_moments` (kernels.py:30-49).  HBM-bound: every K and V token
// row is read exactly once with 16-byte loads (through the index for indexed
// windows); the outputs are written in the layouts the attention kernels use:
//   ctiles [B, H, NCT, 2, 64 D] BF16 block centroids, 64 key blocks per tile,
//                          as a swizzled K / V tile pair (TileLayout);
//                          NCT = ceil(NKB / 64), zero beyond the last block
//   tiles  [B, H, NKB, 2, 64 D] K and V token tiles per key block, only for
//                          keys the attention kernels cannot DMA row by row
//                          straight from K and V (indexed or ragged windows,
//                          fewer than 64 keys)
// Both are streamed into LDS by the attention kernels with DMA.
// Sums follow torch's CPU outer-reduction order (16-row sequential chunks,
// folded in order), so the FP32 means and the BF16-rounded centroids equal the
// reference oracle's `x[:, i:i+64].float().mean(1)` bit for bit.
#include "sol_device.h"
#include "sol_internal.h"

// This file is compiled with -ffp-contract=off: every product and sum below is
// rounded on its own, as in torch's CPU reduction (a fused sq - m*m would
// differ in the last bit).

namespace sol {

// Two workgroup forms, both covering one 16-block chunk per workgroup:
// - NW = 4 waves, each pooling 4 blocks in turn (large grids), each keeping
//   16 rows x 16 bytes per lane in flight, with non-temporal loads (K and V
//   are streamed once here).  Two waves per SIMD: at 84,672 tokens x 24
//   heads the read-only pass measured 0.231 ms at one wave per SIMD, 0.207
//   at two, 0.210 at three, and 0.172 with two and non-temporal loads;
//   issuing the next block's loads before summing the current one (two
//   blocks in flight per wave) did not help (0.210).
// - NW = 16 / BPI waves, one block (D = 128) or two (D = 64) each, all in
//   flight at once (grids too small to fill the GPU, where the four
//   sequential rounds of the first form are the whole run time).
template <int D, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(1, NW == 4 ? 2 : NW / 4)))
void pool_kv_kernel(PoolParams p) {
  constexpr int DC = D / 8;          // 16-byte chunks per token row
  constexpr int LPB = DC * 4;        // lanes per key block: 4 chunks of 16 rows
  constexpr int BPI = kWave / LPB;   // key blocks per wave iteration
  constexpr int NT = NW * kWave;
  constexpr int ITERS = kPoolChunk / (NW * BPI);  // iterations per wave
  static_assert(ITERS * NW * BPI == kPoolChunk, "a workgroup covers one chunk");
  using TL = TileLayout<D>;
  __shared__ __align__(16) uint16_t cent[kPoolChunk][D];

  const bool is_v = blockIdx.y != 0;
  const TokenRows src = is_v ? p.v : p.k;
  // Heads vary fastest over the grid: the workgroups in flight together read
  // whole token rows (all heads of the same tokens), so the DRAM pages they
  // open are read through instead of in 2 D-byte pieces far apart in time.
  const int c = blockIdx.x / (p.B * p.H);
  const int bh = blockIdx.x % (p.B * p.H);
  const int h = bh % p.H, b = bh / p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane / LPB, r4 = (lane % LPB) / DC, dc = lane % DC;
  const int tk = batch_tokens(p.klen, b, p.Tk);  // this entry's key tokens
  const int nkb = (tk + kBlock - 1) / kBlock;

#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int jb = (wave * ITERS + it) * BPI + sub;  // block inside this chunk
    const int j = c * kPoolChunk + jb;
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = 0.f;
    int len = 0;
    if (j < nkb) {
      len = min(kBlock, tk - kBlock * j);
      u32x4 x[16];
      load_rows16<16, true>(src, b, kBlock * j + 16 * r4, kBlock * j + len - 1, h, 8 * dc, x);
      if (p.tiles) {
        // Attention-ready tiles in the LDS image layout (zero past the end),
        // for keys the attention kernels cannot DMA row by row.
        uint16_t* tile = p.tiles + ((int64_t(b) * p.H + h) * p.NKB + j) * 2 * TL::kElems;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = 16 * r4 + i;
          *reinterpret_cast<u32x4*>(tile + (is_v ? TL::kElems + TL::v_offset(row, dc) : TL::k_offset(row, dc))) = x[i];
        }
      }
      // Sequential accumulation inside the 16-row chunk (torch order).
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (16 * r4 + i < len) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = x[i][e >> 1];
            s[e] = __fadd_rn(s[e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)));
          }
        }
      }
    }
    float t1[8], t2[8], t3[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      t1[e] = __shfl(s[e], lane + DC);
      t2[e] = __shfl(s[e], lane + 2 * DC);
      t3[e] = __shfl(s[e], lane + 3 * DC);
    }
    if (r4 == 0) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float m0 = 0.f, m1 = 0.f;
        if (len > 0) {
          const float a0 = __fadd_rn(__fadd_rn(__fadd_rn(s[e], t1[e]), t2[e]), t3[e]);
          const float a1 = __fadd_rn(__fadd_rn(__fadd_rn(s[e + 1], t1[e + 1]), t2[e + 1]), t3[e + 1]);
          m0 = __fdiv_rn(a0, float(len));
          m1 = __fdiv_rn(a1, float(len));
        }
        o[e >> 1] = pack_bf16x2(m0, m1);
      }
      *reinterpret_cast<u32x4*>(&cent[jb][8 * dc]) = o;
    }
  }
  __syncthreads();

  const int64_t head = int64_t(b) * p.H + h;
  if (!p.ctiles) return;  // tiles only (dense path)
  // Centroid tiles: 64 consecutive key blocks per tile, laid out like a K / V
  // tile pair.  This chunk fills rows r0 .. r0 + 15 of tile ct.
  const int ct = (c * kPoolChunk) / kBlock;
  const int r0 = (c * kPoolChunk) % kBlock;
  uint16_t* ctile = p.ctiles + (head * p.NCT + ct) * 2 * TL::kElems;
  if (!is_v) {
    if (tid < kPoolChunk * DC) {
      const int jb = tid / DC, cc = tid % DC;
      *reinterpret_cast<u32x4*>(ctile + TL::k_offset(r0 + jb, cc)) =
          *reinterpret_cast<const u32x4*>(&cent[jb][8 * cc]);
    }
    // Chunk partial sums of the BF16 centroids and their squares (moments).
    const int nch = (p.NKB + kPoolChunk - 1) / kPoolChunk;  // layout stride
    if (p.ksum && c * kPoolChunk < nkb && tid < D) {
      const int rows = min(kPoolChunk, nkb - c * kPoolChunk);
      float s1 = 0.f, s2 = 0.f;
      for (int jb = 0; jb < rows; ++jb) {
        const float x = bf16_bits_to_f32(cent[jb][tid]);
        s1 = __fadd_rn(s1, x);
        s2 = __fadd_rn(s2, __fmul_rn(x, x));
      }
      float* dst = p.ksum + ((head * nch + c) * 2) * D;
      dst[tid] = s1;
      dst[D + tid] = s2;
      if (p.NKB <= kPoolChunk) {
        // One chunk per entry: moments_kernel's fold reduces to these two
        // divisions, so the moments are written here and its launch is
        // skipped (launch_pool).
        const float n = float(nkb);
        const float m = __fdiv_rn(s1, n);
        const float v = __fdiv_rn(s2, n) - m * m;
        p.mean[head * D + tid] = m;
        p.var[head * D + tid] = v > 0.f ? v : 0.f;
      }
    }
  } else if (tid < kPoolChunk * DC) {
    const int jb = tid / DC, cc = tid % DC;
    *reinterpret_cast<u32x4*>(ctile + TL::kElems + TL::v_offset(r0 + jb, cc)) =
        *reinterpret_cast<const u32x4*>(&cent[jb][8 * cc]);
  }
}

// Waves of the wide form: 16 blocks, BPI = 64 / (D / 2) blocks per wave.
template <int D>
constexpr int kWideWaves = kPoolChunk / (kWave / (D / 2));

// One workgroup per (batch, head): fold the 16-block chunk sums in torch's
// cascade order.  The fold is sequential only between 256-block groups: the
// sums of 16 consecutive chunks (what torch's level-1 accumulator holds when it
// carries) are formed in parallel, then one thread per feature folds them.
constexpr int kMomentThreads = 512;
constexpr int kGroupsPerPass = 32;

template <int D>
__global__ __launch_bounds__(kMomentThreads) void moments_kernel(const float* __restrict__ ksum,
                                                                 float* __restrict__ mean,
                                                                 float* __restrict__ var,
                                                                 const int32_t* __restrict__ klen,
                                                                 int tk_all, int nkb_all, int heads) {
  constexpr int G = kMomentThreads / D;  // threads per feature
  __shared__ float gs[2][kGroupsPerPass][D];
  const int bh = blockIdx.x, d = threadIdx.x % D, gi = threadIdx.x / D;
  const int nkb = (batch_tokens(klen, bh / heads, tk_all) + kBlock - 1) / kBlock;  // this entry's blocks
  const int nch = (nkb_all + kPoolChunk - 1) / kPoolChunk;  // layout stride of the chunk sums
  const int full_chunks = nkb / kPoolChunk;
  const int full_groups = full_chunks / 16;
  const float* base = ksum + int64_t(bh) * nch * 2 * D;
  float a2[2] = {0.f, 0.f}, a3[2] = {0.f, 0.f};
  int rows = 0;
  for (int g0 = 0; g0 < full_groups; g0 += kGroupsPerPass) {
    const int ng = min(kGroupsPerPass, full_groups - g0);
    for (int m = gi; m < ng; m += G) {
      const int c0 = (g0 + m) * 16;
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s1 = s1 + base[(2 * (c0 + i)) * D + d];
        s2 = s2 + base[(2 * (c0 + i) + 1) * D + d];
      }
      gs[0][m][d] = s1;
      gs[1][m][d] = s2;
    }
    __syncthreads();
    if (gi == 0) {
      for (int m = 0; m < ng; ++m) {
        rows += 256;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          a2[w] = a2[w] + gs[w][m][d];
          if ((rows & 0xF00) == 0) {
            a3[w] = a3[w] + a2[w];
            a2[w] = 0.f;
          }
        }
      }
    }
    __syncthreads();
  }
  if (gi != 0) return;
  float a1[2] = {0.f, 0.f}, rem[2] = {0.f, 0.f};
  for (int c = full_groups * 16; c < full_chunks; ++c) {
    a1[0] = a1[0] + base[(2 * c) * D + d];
    a1[1] = a1[1] + base[(2 * c + 1) * D + d];
  }
  if (full_chunks * kPoolChunk < nkb) {
    rem[0] = base[(2 * full_chunks) * D + d];
    rem[1] = base[(2 * full_chunks + 1) * D + d];
  }
  const float n = float(nkb);
  const float m = __fdiv_rn(((rem[0] + a1[0]) + a2[0]) + a3[0], n);
  const float sq = __fdiv_rn(((rem[1] + a1[1]) + a2[1]) + a3[1], n);
  const float v = sq - m * m;
  mean[int64_t(bh) * D + d] = m;
  var[int64_t(bh) * D + d] = v > 0.f ? v : 0.f;
}

// Grids of at most this many chunk workgroups (K and V together) use the
// wide form: they leave most CUs idle, so latency, not bandwidth, sets their
// time.
constexpr int64_t kWidePoolGroups = 512;

hipError_t launch_pool(const PoolParams& p, int D, hipStream_t stream) {
  const dim3 grid(unsigned(p.B) * p.H * p.NCHP, 2);
  const bool wide = 2 * int64_t(p.B) * p.H * p.NCHP <= kWidePoolGroups;
  if (D == 128) {
    if (wide)
      hipLaunchKernelGGL((pool_kv_kernel<128, kWideWaves<128>>), grid, dim3(kWideWaves<128> * kWave), 0, stream, p);
    else
      hipLaunchKernelGGL((pool_kv_kernel<128, 4>), grid, dim3(256), 0, stream, p);
  } else {
    if (wide)
      hipLaunchKernelGGL((pool_kv_kernel<64, kWideWaves<64>>), grid, dim3(kWideWaves<64> * kWave), 0, stream, p);
    else
      hipLaunchKernelGGL((pool_kv_kernel<64, 4>), grid, dim3(256), 0, stream, p);
  }
  hipError_t err = hipGetLastError();
  // Single-chunk keys had their moments written by the pooling kernel.
  if (err != hipSuccess || !p.ksum || !p.ctiles || p.NKB <= kPoolChunk) return err;
  if (D == 128)
    hipLaunchKernelGGL(moments_kernel<128>, dim3(p.B * p.H), dim3(kMomentThreads), 0, stream,
                       p.ksum, p.mean, p.var, p.klen, p.Tk, p.NKB, p.H);
  else
    hipLaunchKernelGGL(moments_kernel<64>, dim3(p.B * p.H), dim3(kMomentThreads), 0, stream,
                       p.ksum, p.mean, p.var, p.klen, p.Tk, p.NKB, p.H);
  return hipGetLastError();
}

}  // namespace sol
