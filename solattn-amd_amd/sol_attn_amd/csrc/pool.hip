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
      // All 16 centroid rows read first (every row of `cent` is written), so
      // the reads overlap; the sums then take the chunk's blocks in order.
      float xs[kPoolChunk];
#pragma unroll
      for (int jb = 0; jb < kPoolChunk; ++jb) xs[jb] = bf16_bits_to_f32(cent[jb][tid]);
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int jb = 0; jb < kPoolChunk; ++jb) {
        if (jb < rows) {
          s1 = __fadd_rn(s1, xs[jb]);
          s2 = __fadd_rn(s2, __fmul_rn(xs[jb], xs[jb]));
        }
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

// Block centroids only, for keys of at most one 16-block chunk whose
// attention launch forms the key moments itself from the centroid tile
// (PoolParams::blocks_only: no chunk sums, no moments, no block tiles, plain
// K / V rows): four waves per workgroup, each pooling one block (D = 128) or
// two (D = 64) as pool_kv_kernel's waves do -- the same loads, the same
// sequential 16-row sums folded in order, the same divisions, so the same
// centroids -- and storing its centroid row straight into the tile, with no
// LDS stage or barrier.  Every row of the tiles is written (zero past the
// last block).  Short launches are latency-bound: the wide form's one
// workgroup of 16 waves per (entry, head, K / V) reads the whole chunk on one
// CU; here 16 workgroups per (entry, head) share it.
template <int D>
__global__ __launch_bounds__(256) void pool_blocks_kernel(PoolParams p) {
  constexpr int DC = D / 8;          // 16-byte chunks per token row
  constexpr int LPB = DC * 4;        // lanes per key block: 4 chunks of 16 rows
  constexpr int BPW = kWave / LPB;   // key blocks per wave
  constexpr int BPG = 4 * BPW;       // key blocks per workgroup
  using TL = TileLayout<D>;
  const bool is_v = blockIdx.y != 0;
  const TokenRows src = is_v ? p.v : p.k;
  const int per_head = p.NCT * kBlock / BPG;
  const int bh = blockIdx.x / per_head, part = blockIdx.x % per_head;
  const int h = bh % p.H, b = bh / p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int sub = lane / LPB, r4 = (lane % LPB) / DC, dc = lane % DC;
  const int j = part * BPG + wave * BPW + sub;  // key block, < NCT * 64
  const int nkb = (p.Tk + kBlock - 1) / kBlock;
  float s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.f;
  int len = 0;
  if (j < nkb) {
    len = min(kBlock, p.Tk - kBlock * j);
    u32x4 x[16];
    load_rows16<16, true>(src, b, kBlock * j + 16 * r4, kBlock * j + len - 1, h, 8 * dc, x);
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
    uint16_t* ctile = p.ctiles + ((int64_t(b) * p.H + h) * p.NCT + j / kBlock) * 2 * TL::kElems;
    const int row = j % kBlock;
    *reinterpret_cast<u32x4*>(ctile + (is_v ? TL::kElems + TL::v_offset(row, dc) : TL::k_offset(row, dc))) = o;
  }
}

// Four heads per workgroup (D = 128, heads a multiple of 4, large grids):
// one 16-block chunk of heads h0 .. h0 + 3, sixteen waves, wave w pooling
// key block w of the chunk.  Lane (hq, dc) reads head h0 + hq's 16-byte
// chunk dc of every row, so one wave instruction covers one token row's four
// heads (1 KiB contiguous for packed heads) instead of one head's row in
// four places 16 rows apart: read on its own, that shape streams the
// 84,672-token K 5.5% faster.  The lane sums its block's 64 rows in torch's
// order itself -- four sequential 16-row sums folded in order -- so the
// centroids, chunk sums and moments are the one-head kernel's bit for bit.
template <int D>
__global__ __launch_bounds__(1024) void pool_kv4_kernel(PoolParams p) {
  constexpr int DC = D / 8;
  static_assert(4 * DC == kWave, "a wave covers four heads' rows");
  using TL = TileLayout<D>;
  __shared__ __align__(16) uint16_t cent[4][kPoolChunk][D];

  const bool is_v = blockIdx.y != 0;
  const TokenRows src = is_v ? p.v : p.k;
  const int hgroups = p.H / 4;
  // (entry, head group) pairs vary fastest, as in the one-head kernel.
  const int c = blockIdx.x / (p.B * hgroups);
  const int bg = blockIdx.x % (p.B * hgroups);
  const int b = bg / hgroups, h0 = (bg % hgroups) * 4;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int hq = lane / DC, dc = lane % DC;
  const int tk = batch_tokens(p.klen, b, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  const int jb = wave;
  const int j = c * kPoolChunk + jb;
  const int len = j < nkb ? min(kBlock, tk - kBlock * j) : 0;
  float tot[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) tot[e] = 0.f;
  if (len > 0) {
    uint16_t* tile = p.tiles ? p.tiles + ((int64_t(b) * p.H + h0 + hq) * p.NKB + j) * 2 * TL::kElems : nullptr;
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
      u32x4 x[16];
      load_rows16<16, true>(src, b, kBlock * j + 16 * q, kBlock * j + len - 1, h0 + hq, 8 * dc, x);
      if (tile) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = 16 * q + i;
          *reinterpret_cast<u32x4*>(tile + (is_v ? TL::kElems + TL::v_offset(row, dc) : TL::k_offset(row, dc))) = x[i];
        }
      }
      float s[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (16 * q + i < len) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = x[i][e >> 1];
            s[e] = __fadd_rn(s[e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)));
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) tot[e] = q == 0 ? s[e] : __fadd_rn(tot[e], s[e]);
    }
  }
  {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float m0 = 0.f, m1 = 0.f;
      if (len > 0) {
        m0 = __fdiv_rn(tot[e], float(len));
        m1 = __fdiv_rn(tot[e + 1], float(len));
      }
      o[e >> 1] = pack_bf16x2(m0, m1);
    }
    *reinterpret_cast<u32x4*>(&cent[hq][jb][8 * dc]) = o;
  }
  __syncthreads();

  if (!p.ctiles) return;  // tiles only (dense path)
  // Centroid tiles: this chunk fills rows r0 .. r0 + 15 of tile ct of each head.
  const int ct = (c * kPoolChunk) / kBlock;
  const int r0 = (c * kPoolChunk) % kBlock;
  {
    const int hh = tid / (kPoolChunk * DC), rest = tid % (kPoolChunk * DC);
    const int r = rest / DC, cc = rest % DC;
    const int64_t head = int64_t(b) * p.H + h0 + hh;
    uint16_t* ctile = p.ctiles + (head * p.NCT + ct) * 2 * TL::kElems;
    *reinterpret_cast<u32x4*>(ctile + (is_v ? TL::kElems + TL::v_offset(r0 + r, cc) : TL::k_offset(r0 + r, cc))) =
        *reinterpret_cast<const u32x4*>(&cent[hh][r][8 * cc]);
  }
  // Chunk partial sums of the BF16 centroids and their squares (moments).
  if (!is_v && p.ksum && c * kPoolChunk < nkb && tid < 4 * D) {
    const int hh = tid / D, f = tid % D;
    const int64_t head = int64_t(b) * p.H + h0 + hh;
    const int nch = (p.NKB + kPoolChunk - 1) / kPoolChunk;  // layout stride
    const int rows = min(kPoolChunk, nkb - c * kPoolChunk);
    float xs[kPoolChunk];
#pragma unroll
    for (int r = 0; r < kPoolChunk; ++r) xs[r] = bf16_bits_to_f32(cent[hh][r][f]);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int r = 0; r < kPoolChunk; ++r) {
      if (r < rows) {
        s1 = __fadd_rn(s1, xs[r]);
        s2 = __fadd_rn(s2, __fmul_rn(xs[r], xs[r]));
      }
    }
    float* dst = p.ksum + ((head * nch + c) * 2) * D;
    dst[f] = s1;
    dst[D + f] = s2;
    if (p.NKB <= kPoolChunk) {
      const float n = float(nkb);
      const float m = __fdiv_rn(s1, n);
      const float v = __fdiv_rn(s2, n) - m * m;
      p.mean[head * D + f] = m;
      p.var[head * D + f] = v > 0.f ? v : 0.f;
    }
  }
}

// Waves of the wide form: 16 blocks, BPI = 64 / (D / 2) blocks per wave.
template <int D>
constexpr int kWideWaves = kPoolChunk / (kWave / (D / 2));

// One workgroup per (batch, head): fold the 16-block chunk sums in torch's
// cascade order.  The fold is sequential only between 256-block groups: the
// sums of 16 consecutive chunks (what torch's level-1 accumulator holds when it
// carries) are formed in parallel, then one thread per feature folds them.
// 1,024 threads: at head_dim 128 eight thread groups, so the 84,672-token
// field's five 256-block group sums and its tail load in one pass (the pool_kv
// call 181.8 -> 181.1 us against 512 threads, alternating on one box).
constexpr int kMomentThreads = 1024;
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
  // The chunks past the last whole 256-block group (at most 15 whole chunks
  // and a partial one) are summed by the last thread group, its loads issued
  // all at once, alongside the group sums instead of after them.
  __shared__ float tail[4][D];
  if (gi == G - 1) {
    const int c_lo = full_groups * 16;
    const bool partial = full_chunks * kPoolChunk < nkb;
    float x[2][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = c_lo + i;
      const bool take = c < full_chunks || (c == full_chunks && partial);
      x[0][i] = take ? base[(2 * c) * D + d] : 0.f;
      x[1][i] = take ? base[(2 * c + 1) * D + d] : 0.f;
    }
    float a1[2] = {0.f, 0.f}, rem[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = c_lo + i;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        if (c < full_chunks) a1[w] = a1[w] + x[w][i];
        else if (c == full_chunks && partial) rem[w] = x[w][i];
      }
    }
    tail[0][d] = a1[0];
    tail[1][d] = a1[1];
    tail[2][d] = rem[0];
    tail[3][d] = rem[1];
  }
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
  __syncthreads();  // the tail sums are published
  if (gi != 0) return;
  const float a1[2] = {tail[0][d], tail[1][d]}, rem[2] = {tail[2][d], tail[3][d]};
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

// Four-head workgroups: large grids at D = 128 with heads in fours.
bool POOL_FOUR_HEADS = true;

hipError_t launch_pool(const PoolParams& p, int D, hipStream_t stream) {
  if (p.blocks_only) {
    const unsigned per_head = unsigned(p.NCT) * kBlock / (D == 128 ? 4 : 8);
    if (D == 128)
      hipLaunchKernelGGL(pool_blocks_kernel<128>, dim3(unsigned(p.B) * p.H * per_head, 2), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL(pool_blocks_kernel<64>, dim3(unsigned(p.B) * p.H * per_head, 2), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  const dim3 grid(unsigned(p.B) * p.H * p.NCHP, 2);
  const bool wide = 2 * int64_t(p.B) * p.H * p.NCHP <= kWidePoolGroups;
  if (D == 128 && !wide && p.H % 4 == 0 && POOL_FOUR_HEADS) {
    hipLaunchKernelGGL(pool_kv4_kernel<128>, dim3(unsigned(p.B) * (p.H / 4) * p.NCHP, 2), dim3(1024), 0, stream, p);
  } else if (D == 128) {
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
  // Single-chunk keys had their moments written by the pooling kernel; with
  // fold_in_attention the attention launch folds the chunk sums itself.
  if (err != hipSuccess || !p.ksum || !p.ctiles || p.NKB <= kPoolChunk || p.fold_in_attention) return err;
  if (D == 128)
    hipLaunchKernelGGL(moments_kernel<128>, dim3(p.B * p.H), dim3(kMomentThreads), 0, stream,
                       p.ksum, p.mean, p.var, p.klen, p.Tk, p.NKB, p.H);
  else
    hipLaunchKernelGGL(moments_kernel<64>, dim3(p.B * p.H), dim3(kMomentThreads), 0, stream,
                       p.ksum, p.mean, p.var, p.klen, p.Tk, p.NKB, p.H);
  return hipGetLastError();
}

}  // namespace sol
