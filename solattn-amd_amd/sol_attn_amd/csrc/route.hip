// Routing of the SOL attention: per (batch entry, query block, head) the
// Eq.15 cutoff and the selected key blocks, as one bit per key block.
//
// Replaces the reference's `_threshold` kernel (src/sol_attn_amd/kernels.py:
// 52-64) and the routing part of `_sol` (kernels.py:118-143): the cutoff
// c = Qc . mu + beta * sqrt(sum Qc^2 var) of the FP32 query-block mean Qc,
// the proxies Qc . Kc_j of every key block's BF16 centroid, selected = proxy
// > c (strict), forced by beta = +-inf, OR the local band, key / query sinks
// and plan protection.  sol_attention_kernel reads the decisions as bitmask
// words, so its centroid and exact passes carry no routing work.
//
// One workgroup per (batch entry, head, 32 consecutive query blocks, range of
// kRouteChunks x 32 key blocks):
//   1. Qc of the 32 blocks: read from the pairing pass (p.qc), or formed here
//      from Q -- each block's rows summed in torch's cascade order (16-row
//      sequential chunks, then ((c0 + c1) + c2) + c3), divided by the valid
//      length: the reference oracle's `_means` (reference.py:13-15).  A
//      launch that forms Qc here has one key range per workgroup.
//   2. Cutoffs, reduced in a fixed order.
//   3. Proxies on the matrix cores: Qc is split exactly into three BF16 terms
//      hi + mid + lo (each term takes the next 8 significant bits, so the sum
//      is Qc to the last bit), and P = Kc [hi mid lo]^T accumulates the
//      products -- BF16 x BF16 products are exact in FP32 -- in FP32.  The
//      proxies are therefore FP32 dot products of Qc and Kc_j, as the
//      reference's FP32 matmul (reference.py:39); only the order of the FP32
//      additions differs, which the routing band covers.  32 key blocks x 32
//      query blocks per MFMA tile (v_mfma_f32_32x32x16_bf16, 24 per tile).
//   4. Decisions and protection; each lane pair (l, l ^ 32) merges its 16 + 16
//      bits into the query block's 32-bit word of the tile's key blocks.
// Masks: uint32 [B, H, NQB, NW], NW = ceil(NKB / 32); bit j of word w is key
// block 32 w + j.  Bits past an entry's key blocks are 0.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr int kRouteThreads = 256;  // four waves
constexpr int kRouteBlocks = 32;    // query blocks per workgroup: the MFMA tile's columns
constexpr int kRouteChunks = 24;    // 32-key-block chunks per workgroup when Qc comes from p.qc
constexpr float kInf = __builtin_huge_valf();

// FP32 -> BF16 bits, round to nearest even, and back.
__device__ __forceinline__ float bf16_rne_f32(float x) {
  return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

template <int D>
__global__ __launch_bounds__(kRouteThreads, 2) void route_kernel(AttnParams p) {
  constexpr int KT = D / 16;
  constexpr int DC = D / 8;          // 16-byte chunks per row
  constexpr int LPB = DC * 4;        // lanes per query block in the mean pass: 4 quarters of 16 rows
  constexpr int BPI = kWave / LPB;   // query blocks per wave iteration
  constexpr int NW = kRouteThreads / kWave;
  constexpr int ITERS = kRouteBlocks / (NW * BPI);
  static_assert(ITERS * NW * BPI == kRouteBlocks, "a workgroup covers its query blocks");
  __shared__ float s_qc[kRouteBlocks][D + 4];
  __shared__ float s_cut[kRouteBlocks];
  __shared__ u32x4 s_bq[3][KT][kWave];  // B operands: hi / mid / lo term, k-step, lane

  const int bh = blockIdx.y;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int qb0 = blockIdx.x * kRouteBlocks;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tk = batch_tokens(p.klen, b, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  const bool finite = p.force == 0;

  if (finite && p.qc) {
    // 1. Query-block means from the pairing pass (every load in flight at once).
    constexpr int kLoads = kRouteBlocks * D / 4 / kRouteThreads;
    f32x4 x[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = tid + u * kRouteThreads;
      const int jb = i / (D / 4), d4 = i % (D / 4);
      const int qb = min(qb0 + jb, p.NQB - 1);  // rows past the last block: never used
      x[u] = *reinterpret_cast<const f32x4*>(p.qc + (head * p.NQB + qb) * D + 4 * d4);
    }
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = tid + u * kRouteThreads;
      const int jb = i / (D / 4), d4 = i % (D / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) s_qc[jb][4 * d4 + e] = qb0 + jb < p.NQB ? x[u][e] : 0.f;
    }
  } else if (finite) {
    // 1. Query-block means.  Lane (quarter r4, chunk dc) sums rows
    // 16 r4 .. 16 r4 + 15 of its block sequentially (rows past the block load
    // as zeros, which add exactly nothing); quarter 0 folds the four sums in
    // order.
    const int sub = lane / LPB, r4 = (lane % LPB) / DC, dc = lane % DC;
#pragma unroll 1
    for (int it = 0; it < ITERS; ++it) {
      const int jb = (wave * ITERS + it) * BPI + sub;
      const int qb = qb0 + jb;
      float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int qlen = 1;
      if (qb < p.NQB) {
        qlen = min(kBlock, p.Tq - kBlock * qb);
        u32x4 x[16];
        load_rows16<16>(p.q, b, kBlock * qb + 16 * r4, kBlock * qb + qlen - 1, h, 8 * dc, x);
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = x[r][e >> 1];
            s[e] = __fadd_rn(s[e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)));
          }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c1 = __shfl(s[e], lane + DC), c2 = __shfl(s[e], lane + 2 * DC), c3 = __shfl(s[e], lane + 3 * DC);
        s[e] = __fadd_rn(__fadd_rn(__fadd_rn(s[e], c1), c2), c3);
      }
      if (r4 == 0)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_qc[jb][8 * dc + e] = qb < p.NQB ? __fdiv_rn(s[e], float(qlen)) : 0.f;
    }
  }
  if (finite) {
    // 2. Cutoffs: c = (a0 + a1) + beta sqrt(g0 + g1), where a_h / g_h sum the
    // terms Qc_d mu_d / Qc_d^2 var_d (full covariance: Qc_d (cov Qc)_d) of
    // feature half h = [64 h, 64 h + 64) over the 64 lanes of a wave by xor
    // shuffles.  Each wave reduces its kRouteBlocks / NW blocks together, so
    // their shuffle chains overlap.
    constexpr int BW = kRouteBlocks / NW;  // blocks per wave
    __syncthreads();
    float mu[2] = {0.f, 0.f}, va[2] = {0.f, 0.f};
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const int d = 64 * part + lane;
      if (d < D) {
        mu[part] = p.mean[head * D + d];
        va[part] = p.cov ? 0.f : p.var[head * D + d];
      }
    }
    float a[BW][2], g[BW][2];
#pragma unroll
    for (int i = 0; i < BW; ++i)
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int jb = wave * BW + i, d = 64 * part + lane;
        a[i][part] = g[i][part] = 0.f;
        if (d < D) {
          const float qm = s_qc[jb][d];
          a[i][part] = qm * mu[part];
          g[i][part] = qm * qm * va[part];
        }
      }
    if (p.cov) {
      // Full covariance (experiment): this feature's term of Qc^T cov Qc,
      // sum_e cov[d][e] Qc_e in feature order.  cov is symmetric bit for bit
      // (covariance_partial_kernel forms entry (d, e) and (e, d) by the same
      // fmas in the same order), so lane d reads column d: one coalesced load
      // per feature e serves the wave's BW blocks.
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        const int d = 64 * part + lane;
        if (d < D) {
          float sq[BW];
#pragma unroll
          for (int i = 0; i < BW; ++i) sq[i] = 0.f;
          const float* col = p.cov + int64_t(head) * D * D + d;
#pragma unroll 4
          for (int e = 0; e < D; ++e) {
            const float c = col[e * D];
#pragma unroll
            for (int i = 0; i < BW; ++i) sq[i] = fmaf(c, s_qc[wave * BW + i][e], sq[i]);
          }
#pragma unroll
          for (int i = 0; i < BW; ++i) g[i][part] = s_qc[wave * BW + i][d] * sq[i];
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
      for (int i = 0; i < BW; ++i)
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          a[i][part] += __shfl_xor(a[i][part], off);
          g[i][part] += __shfl_xor(g[i][part], off);
        }
    if (lane == 0)
#pragma unroll
      for (int i = 0; i < BW; ++i) {
        const float quad = g[i][0] + g[i][1];  // the full quadratic form may round below 0
        s_cut[wave * BW + i] = (a[i][0] + a[i][1]) + p.beta * sqrtf(p.cov ? fmaxf(quad, 0.f) : quad);
      }
    __syncthreads();
  }
  const int col = lane & 31, hh = lane >> 5;
  const int qb = qb0 + col;  // this lane's query block (MFMA column)
  const bool qlive = qb < p.NQB;
  if (p.dbg_cutoff && qlive && hh == 0 && wave == 0 && blockIdx.z == 0)
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb) * p.H + h] = finite ? s_cut[col] * p.scale : kInf;  // beta = +inf

  // 3. The B operand of every tile, built once per workgroup in LDS: lane
  // (col, hh) of k-step ks takes features 16 ks + 8 hh .. + 7 of Qc[qb0 +
  // col] as hi / mid / lo BF16 terms (the waves share the k-steps).
  if (finite) {
    for (int ks = wave; ks < KT; ks += NW) {
      u32x4 w[3];
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float x[2], t[3][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          x[u] = s_qc[col][16 * ks + 8 * hh + i + u];
          t[0][u] = bf16_rne_f32(x[u]);
          const float r1 = __fsub_rn(x[u], t[0][u]);
          t[1][u] = bf16_rne_f32(r1);
          t[2][u] = bf16_rne_f32(__fsub_rn(r1, t[1][u]));
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) w[k][i >> 1] = pack_bf16x2(t[k][0], t[k][1]);
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) s_bq[k][ks][lane] = w[k];
    }
    __syncthreads();
  }
  const float cut = finite ? s_cut[col] : 0.f;
  const uint16_t* kc_head = p.ctiles + head * p.NCT * (2 * kBlock * D);
  const int64_t dbg_row = ((int64_t(b) * p.NQB + qb) * p.H + h) * p.NKB;
  // This workgroup's chunks of 32 key blocks: all of them, or kRouteChunks
  // from blockIdx.z kRouteChunks on when the means come from p.qc.
  const int nchunk = (nkb + 31) / 32;
  const int kc_lo = p.qc ? int(blockIdx.z) * kRouteChunks : 0;
  const int kc_hi = p.qc ? min(nchunk, kc_lo + kRouteChunks) : nchunk;
  // A operand of chunk kc: key block 32 kc + col, features 16 ks + 8 hh .. + 7,
  // from the K half of its centroid tile (rows past the sequence are zero).
  auto load_chunk = [&](int kc, u32x4 (&ka)[KT]) {
    const int r = 32 * kc + col;
    const uint16_t* tile = kc_head + int64_t(r >> 6) * (2 * kBlock * D);
#pragma unroll
    for (int ks = 0; ks < KT; ++ks) ka[ks] = load16(tile + TileLayout<D>::k_offset(r & 63, 2 * ks + hh));
  };
  // Chunks kc_lo + wave, + NW, ...: two operand buffers take turns, the next
  // chunk's loads in flight while the current chunk is on the matrix cores.
  u32x4 kbuf[2][KT];
  int kc = kc_lo + wave;
  if (finite && kc < kc_hi) load_chunk(kc, kbuf[0]);
  for (int it = 0; kc < kc_hi; kc += NW, ++it) {
    const int j0 = 32 * kc;
    f32x16 acc = zero16();
    if (finite) {
      auto mfmas = [&](u32x4 (&cur)[KT], u32x4 (&nxt)[KT]) {
        if (kc + NW < kc_hi) load_chunk(kc + NW, nxt);
#pragma unroll
        for (int ks = 0; ks < KT; ++ks)
#pragma unroll
          for (int k = 0; k < 3; ++k) acc = mfma32x32x16(as_bf16x8(cur[ks]), as_bf16x8(s_bq[k][ks][lane]), acc);
      };
      if (it & 1)
        mfmas(kbuf[1], kbuf[0]);
      else
        mfmas(kbuf[0], kbuf[1]);
    }
    // Decisions as bits (row r of the tile: key block j0 + r), branch-free;
    // the plan's protection and the diagnostics follow behind uniform
    // branches.  Lane half hh holds rows 8 (e / 4) + 4 hh + e % 4.
    const int jh = j0 + 4 * hh;
    const bool all_rows = qb < p.q_sink_blocks;
    uint32_t bits = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 8 * (e >> 2) + 4 * hh + (e & 3);
      const int j = jh + 8 * (e >> 2) + (e & 3);
      const bool sel = (finite && acc[e] > cut) || all_rows || j < p.kv_sink_blocks ||
                       (p.local_blocks >= 0 && abs(j - qb) <= p.local_blocks);
      bits |= uint32_t(sel) << row;
    }
    if (p.protection && qlive) {
      const uint8_t* prow = p.protection + (int64_t(b) * p.NQB + qb) * p.NKB;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 8 * (e >> 2) + 4 * hh + (e & 3);
        const int j = jh + 8 * (e >> 2) + (e & 3);
        bits |= uint32_t(j < nkb && prow[min(j, nkb - 1)] != 0) << row;
      }
    }
    // Only key blocks of the entry, and only live query blocks.
    const int nvalid = min(max(nkb - j0, 0), 32);
    bits &= qlive ? (nvalid == 32 ? ~0u : ((1u << nvalid) - 1u)) : 0u;
    if ((p.dbg_proxy || p.dbg_selected) && qlive) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 8 * (e >> 2) + 4 * hh + (e & 3);
        const int j = jh + 8 * (e >> 2) + (e & 3);
        if (j < nkb) {
          if (p.dbg_proxy && finite) p.dbg_proxy[dbg_row + j] = acc[e] * p.scale;
          if (p.dbg_selected) p.dbg_selected[dbg_row + j] = uint8_t((bits >> row) & 1u);
        }
      }
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
    const uint32_t word = sw[0] | sw[1];
    if (qlive && hh == 0) p.mask[(head * p.NQB + qb) * p.NW + kc] = word;
  }
}

}  // namespace

hipError_t launch_route(const AttnParams& p, int D, hipStream_t stream) {
  const int nchunk = (p.NKB + 31) / 32;
  const unsigned splits = p.qc ? unsigned((nchunk + kRouteChunks - 1) / kRouteChunks) : 1u;
  const dim3 grid(unsigned((p.NQB + kRouteBlocks - 1) / kRouteBlocks), unsigned(p.B * p.H), splits);
  if (D == 128)
    hipLaunchKernelGGL(route_kernel<128>, grid, dim3(kRouteThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(route_kernel<64>, grid, dim3(kRouteThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
