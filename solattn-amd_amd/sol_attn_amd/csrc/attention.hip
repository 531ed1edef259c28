// Fused SOL routing + attention, and the dense flash-attention control, for gfx950.
//
// Replaces the reference's `_threshold` (src/sol_attn_amd/kernels.py:52-64),
// `_sol` (kernels.py:101-182) and `_dense` (kernels.py:67-98).
//
// SOL workgroup = one 64-query block of one (batch, head), 4 waves.  Wave w
// owns queries 32*(w&1) .. +31 and key half (w>>1) of every 64-key block, with
// its own FP32 online-softmax state; the two key halves are merged at the end.
//   1. Q tile -> LDS -> register fragments (MFMA B operand of S^T = K Q^T)
//   2. FP32 query mean (torch cascade order) and the Eq.15 cutoff
//      c = Qc.mu + beta * sqrt(sum Qc^2 var)                    (kernels.py:58-63)
//   3. routing: proxy_j = Qc . Kc_j (= mean over the block's rows of q_r . Kc_j),
//      selected = proxy > c, OR sink / local / plan protection; decisions live
//      in an LDS bitmask, never in HBM                          (kernels.py:129-143)
//   4. centroid correction for unselected blocks, 32 centroids per MFMA tile
//      (tiles alternate between the key-half waves):
//      w = exp2(s - m) * valid_len, O^T += Vc^T bf16(w)^T        (kernels.py:145-158)
//   5. exact blocks in ascending order: the pooling pass's swizzled K / V^T
//      tiles stream into a double-buffered LDS ring with global_load_lds DMA
//      (block i+1 lands while block i is on the matrix cores);
//      S^T = K Q^T, online softmax, O^T += V^T bf16(P)^T           (kernels.py:159-178)
//   6. merge the key halves, O = acc / den, BF16 store, exact count (kernels.py:179-182)
// Every contribution shares the FP32 online-softmax state of its wave, in log2
// units; empty states use max 0 for the rescale (kernels.py:148-150).
// The dense control runs step 5 over every key block, 128 queries per
// workgroup (4 waves x 32 queries, full 64-key blocks per wave).
#include "sol_device.h"
#include "sol_internal.h"

#define SOL_LDS __attribute__((address_space(3)))

namespace sol {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

constexpr int kXcds = 8;

// Workgroup ids are dealt round-robin over the 8 XCDs.  The id -> (head, query
// tile) map keeps every XCD on the SAME head at the same time, each on its own
// contiguous 1/8 slice of the query tiles: neighbouring tiles share that XCD's
// L2, and the tiles of one head (43 MB at 84,672 tokens) are the whole live
// set of the memory-side cache.  Grid = 8 * heads * slice; ids past the end of
// a slice return -1 (idle workgroup).
struct TileTask {
  int bh, tile;
};

__device__ __forceinline__ TileTask xcd_task(int i, int ntiles) {
  const int slice = (ntiles + kXcds - 1) / kXcds;
  const int xcd = i % kXcds, k = i / kXcds;
  const int tile = xcd * slice + k % slice;
  return TileTask{tile < ntiles ? k / slice : -1, tile};
}

__host__ __device__ inline unsigned xcd_grid(int heads, int ntiles) {
  return unsigned(kXcds) * unsigned(heads) * unsigned((ntiles + kXcds - 1) / kXcds);
}

template <int D>
struct Shape {
  static constexpr int KS = D + 8;   // Q staging row stride (elements)
  static constexpr int DC = D / 8;   // 16-byte chunks per row
  static constexpr int KT = D / 16;  // MFMA k-steps over the head dimension
  static constexpr int DT = D / 32;  // 32-row output tiles over the head dimension
  static constexpr int TILE = 2 * kBlock * D;  // K + V^T tile elements per key block
};

// One wave's FP32 online-softmax state for its 32 queries (one per lane pair).
template <int D>
struct State {
  f32x16 acc[Shape<D>::DT];  // O^T: rows = features, column = this lane's query
  float m;                   // running max, log2 units (-inf: nothing yet)
  float den;                 // partial denominator over this lane's key rows
};

template <int D>
__device__ __forceinline__ void state_init(State<D>& st) {
#pragma unroll
  for (int dt = 0; dt < Shape<D>::DT; ++dt) st.acc[dt] = zero16();
  st.m = kNegInf;
  st.den = 0.f;
}

// Online-softmax update with the scores s[0..NS) (log2 units, -inf = absent).
// Returns the probabilities in s.
template <int D, int NS>
__device__ __forceinline__ void softmax_update(State<D>& st, f32x16 (&s)[NS]) {
  float mx = kNegInf;
#pragma unroll
  for (int t = 0; t < NS; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mnew = fmaxf(st.m, mx);
  const float safe = mnew == kNegInf ? 0.f : mnew;
  const float alpha = fast_exp2(st.m - safe);
  float lsum = 0.f;
#pragma unroll
  for (int t = 0; t < NS; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = fast_exp2(s[t][e] - safe);
      s[t][e] = pe;
      lsum += pe;
    }
  st.den = st.den * alpha + lsum;
  st.m = mnew;
#pragma unroll
  for (int dt = 0; dt < Shape<D>::DT; ++dt) st.acc[dt] *= alpha;
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& s, int base) {
  u32x4 pb;
#pragma unroll
  for (int i = 0; i < 4; ++i) pb[i] = pack_bf16x2(s[base + 2 * i], s[base + 2 * i + 1]);
  return as_bf16x8(pb);
}

// 16-byte global -> LDS DMA per lane: lane l's bytes land at lds_base + 16 l.
// Issued as inline assembly so that the compiler does not drain the vector
// memory counter before every LDS read (it cannot tell the ring's two buffers
// apart); completion is awaited explicitly with wait_vmcnt before the barrier.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_base);  // wave-uniform by construction
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(base), "v"(src) : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((SOL_LDS const void*)p));
}

// Issue the DMA of one K + V^T tile pair (contiguous in HBM) into an LDS buffer.
template <int D, int NT>
__device__ __forceinline__ void tile_dma(const uint16_t* src, uint16_t* dst, int wave, int lane) {
  constexpr int kChunks = Shape<D>::TILE / 8;   // 16-byte chunks per tile pair
  constexpr int kRounds = kChunks / NT;
  static_assert(kChunks % NT == 0, "tile pair must split evenly over the workgroup");
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int chunk = r * NT + wave * kWave;  // first chunk of this wave's 1 KB piece
    dma16(src + (chunk + lane) * 8, lds_address(dst + chunk * 8));
  }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without a memory fence: LDS DMA completion is awaited
// explicitly with s_waitcnt vmcnt, so the in-flight prefetch of the next tile
// is not drained here.  The "memory" clobber keeps LDS accesses on their side.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Exact 64-key block from an LDS tile pair: key halves [kh0, kh0 + NH).
template <int D, int NH>
__device__ __forceinline__ void exact_block(const uint16_t* buf, int j, int tk, float scale_log2,
                                            int kh0, const bf16x8 (&qf)[Shape<D>::KT], int col,
                                            int hh, State<D>& st) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  const uint16_t* kt_lds = buf;
  const uint16_t* vt_lds = buf + TL::kElems;
  f32x16 s[NH];
#pragma unroll
  for (int t = 0; t < NH; ++t) {
    s[t] = zero16();
    const int row = 32 * (kh0 + t) + col;
#pragma unroll
    for (int ks = 0; ks < S::KT; ++ks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(kt_lds + TL::k_offset(row, 2 * ks + hh));
      s[t] = mfma32x32x16(as_bf16x8(a), qf[ks], s[t]);
    }
  }
  const bool tail = (j + 1) * kBlock > tk;
#pragma unroll
  for (int t = 0; t < NH; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = s[t][e] * scale_log2;
      if (tail && j * kBlock + 32 * (kh0 + t) + 8 * (e >> 2) + 4 * hh + (e & 3) >= tk) v = kNegInf;
      s[t][e] = v;
    }
  softmax_update<D, NH>(st, s);
#pragma unroll
  for (int t = 0; t < NH; ++t)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const bf16x8 b = pack8(s[t], 8 * c);
      const int g = 8 * (kh0 + t) + 4 * c + hh;  // 4-key group of keys 32(kh0+t) + 16c + 4hh
#pragma unroll
      for (int dt = 0; dt < S::DT; ++dt) {
        const int d = dt * 32 + col;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vt_lds + TL::vt_offset(d, g));
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vt_lds + TL::vt_offset(d, g + 2));
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        st.acc[dt] = mfma32x32x16(as_bf16x8(a), b, st.acc[dt]);
      }
    }
}

template <int D>
__device__ __forceinline__ void store_output(const AttnParams& p, int b, int h, int t, int hh,
                                             const State<D>& st) {
  using S = Shape<D>;
  const float den = st.den + __shfl_xor(st.den, 32);
  if (t >= p.Tq) return;
  uint16_t* orow = p.out + ((int64_t(b) * p.Tq + t) * p.H + h) * D;
#pragma unroll
  for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      u32x2 o;
      o[0] = pack_bf16x2(__fdiv_rn(st.acc[dt][4 * k4], den), __fdiv_rn(st.acc[dt][4 * k4 + 1], den));
      o[1] = pack_bf16x2(__fdiv_rn(st.acc[dt][4 * k4 + 2], den), __fdiv_rn(st.acc[dt][4 * k4 + 3], den));
      *reinterpret_cast<u32x2*>(orow + dt * 32 + 8 * k4 + 4 * hh) = o;
    }
}

// Stream a sequence of exact blocks through the double-buffered LDS ring.
// `next()` yields block ids in order and is evaluated identically by every
// thread (uniform control flow around the barriers).
template <int D, int NT, int NH, typename Next>
__device__ __forceinline__ void exact_stream(const uint16_t* head_tiles, uint16_t* ring, int count,
                                             Next next, int tk, float scale_log2, int kh0,
                                             const bf16x8 (&qf)[Shape<D>::KT], int wave, int lane,
                                             State<D>& st) {
  using S = Shape<D>;
  constexpr int kRounds = S::TILE / 8 / NT;
  if (count <= 0) return;
  const int col = lane & 31, hh = lane >> 5;
  int cur = next();
  tile_dma<D, NT>(head_tiles + int64_t(cur) * S::TILE, ring, wave, lane);
  for (int i = 0; i < count; ++i) {
    const int nxt = i + 1 < count ? next() : -1;
    if (nxt >= 0) {
      tile_dma<D, NT>(head_tiles + int64_t(nxt) * S::TILE, ring + ((i + 1) & 1) * S::TILE, wave, lane);
      wait_vmcnt<kRounds>();
    } else {
      wait_vmcnt<0>();
    }
    ring_barrier();
    exact_block<D, NH>(ring + (i & 1) * S::TILE, cur, tk, scale_log2, kh0, qf, col, hh, st);
    ring_barrier();
    cur = nxt;
  }
}

// Iterates the set bits of an LDS bitmask in ascending order.
struct MaskCursor {
  const uint32_t* mask;
  int word;
  uint32_t bits;
  __device__ __forceinline__ int operator()() {
    while (bits == 0) bits = mask[++word];
    const int j = word * 32 + __builtin_ctz(bits);
    bits &= bits - 1u;
    return j;
  }
};

struct RangeCursor {
  int j;
  __device__ __forceinline__ int operator()() { return j++; }
};

}  // namespace

// __launch_bounds__(256, 2): at least two waves per SIMD (<= 256 registers).
template <int D>
__global__ __launch_bounds__(256, 2) void sol_attention_kernel(AttnParams p) {
  using S = Shape<D>;
  constexpr int NT = 256;
  __shared__ __align__(16) uint16_t ring[2 * S::TILE];  // Q staging / tile ring / merge scratch
  __shared__ float s_qm[D];
  __shared__ float s_red[8];
  __shared__ uint32_t s_mask[kMaxKeyBlocks / 32];

  const TileTask task = xcd_task(blockIdx.x, p.NQB);
  if (task.bh < 0) return;
  const int qb = task.tile;
  const int bh = task.bh;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int q0 = qb * kBlock;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, hh = lane >> 5;
  const int qh = wave & 1, kh = wave >> 1;

  // 1. Q tile -> LDS -> fragments.
  for (int idx = tid; idx < kBlock * S::DC; idx += NT) {
    const int r = idx / S::DC, c = idx % S::DC;
    const int t = q0 + r;
    const u32x4 x = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(ring + r * S::KS + 8 * c) = x;
  }
  __syncthreads();
  bf16x8 qf[S::KT];
  const int myq = 32 * qh + col;
#pragma unroll
  for (int ks = 0; ks < S::KT; ++ks)
    qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(ring + myq * S::KS + ks * 16 + 8 * hh));

  // 2. Query mean and cutoff.
  float cut = 0.f;
  if (p.force == 0) {
    const int qlen = min(kBlock, p.Tq - q0);
    if (tid < D) {
      float tot = 0.f;
      for (int c = 0; c < 4; ++c) {
        float s = 0.f;
        for (int i = 0; i < 16; ++i) {
          const int r = 16 * c + i;
          if (r < qlen) s = __fadd_rn(s, bf16_bits_to_f32(ring[r * S::KS + tid]));
        }
        tot = __fadd_rn(tot, s);
      }
      s_qm[tid] = __fdiv_rn(tot, float(qlen));
    }
    __syncthreads();
    float a = 0.f, g = 0.f;
    if (tid < D) {
      const float qm = s_qm[tid];
      a = qm * p.mean[head * D + tid];
      g = qm * qm * p.var[head * D + tid];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      a += __shfl_xor(a, off);
      g += __shfl_xor(g, off);
    }
    if (lane == 0) {
      s_red[wave] = a;
      s_red[4 + wave] = g;
    }
    __syncthreads();
    const float mu = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    const float sg = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
    cut = mu + p.beta * sqrtf(sg);
  }
  if (p.dbg_cutoff && tid == 0)
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb) * p.H + h] =
        p.force == 0 ? cut * p.scale : (p.force == 1 ? kNegInf : -kNegInf);

  // 3. Routing decisions -> LDS bitmask.
  const int64_t dbg_row = ((int64_t(b) * p.NQB + qb) * p.H + h) * p.NKB;
  for (int j0 = 0; j0 < p.NKB; j0 += NT) {
    const int j = j0 + tid;
    bool sel = false;
    if (j < p.NKB) {
      if (p.force == 1) {
        sel = true;
      } else if (p.force == 0) {
        const uint16_t* kr = p.kc + (head * p.NKB + j) * D;
        float proxy = 0.f;
#pragma unroll
        for (int c = 0; c < S::DC; ++c) {
          const u32x4 x = load16(kr + 8 * c);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = x[e >> 1];
            proxy = fmaf(s_qm[8 * c + e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)), proxy);
          }
        }
        sel = proxy > cut;
        if (p.dbg_proxy) p.dbg_proxy[dbg_row + j] = proxy * p.scale;
      }
      sel = sel || (p.local_blocks >= 0 && abs(j - qb) <= p.local_blocks) ||
            j < p.kv_sink_blocks || qb < p.q_sink_blocks;
      if (p.protection) sel = sel || p.protection[(int64_t(b) * p.NQB + qb) * p.NKB + j] != 0;
      if (p.dbg_selected) p.dbg_selected[dbg_row + j] = sel ? 1 : 0;
    }
    const uint64_t bal = __ballot(sel);
    if (lane == 0) {
      s_mask[(j0 + wave * 64) / 32] = uint32_t(bal);
      s_mask[(j0 + wave * 64) / 32 + 1] = uint32_t(bal >> 32);
    }
  }
  __syncthreads();
  const int nwords = (p.NKB + 31) / 32;
  int nsel = 0;
  for (int w = 0; w < nwords; ++w) nsel += __builtin_popcount(s_mask[w]);
  if (p.counts && tid == 0) p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = nsel;

  State<D> st;
  state_init(st);

  // 4. Centroid correction, 32-centroid tiles split between the key halves.
  if (p.force != 1) {
    const uint16_t* kc = p.kc + head * p.NKB * D;
    const uint16_t* vct = p.vct + head * D * p.NKBP;
    for (int t0 = 32 * kh; t0 < p.NKB; t0 += 64) {
      const int nvalid = min(32, p.NKB - t0);
      const uint32_t validw = nvalid == 32 ? 0xFFFFFFFFu : ((1u << nvalid) - 1u);
      const uint32_t apw = validw & ~s_mask[t0 >> 5];
      if (apw == 0) continue;  // wave-uniform
      f32x16 sc[1];
      sc[0] = zero16();
      const bool row_ok = t0 + col < p.NKB;
#pragma unroll
      for (int ks = 0; ks < S::KT; ++ks) {
        const u32x4 a = row_ok ? load16(kc + int64_t(t0 + col) * D + ks * 16 + 8 * hh) : zero_u32x4();
        sc[0] = mfma32x32x16(as_bf16x8(a), qf[ks], sc[0]);
      }
      float mx = kNegInf;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
        sc[0][e] = ((apw >> r) & 1u) ? sc[0][e] * p.scale_log2 : kNegInf;
        mx = fmaxf(mx, sc[0][e]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(st.m, mx);
      const float safe = mnew == kNegInf ? 0.f : mnew;
      const float alpha = fast_exp2(st.m - safe);
      float wsum = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
        // weight = exp2(s - m) * valid length; 0 for selected / padding blocks
        const float w = ((apw >> r) & 1u)
                            ? fast_exp2(sc[0][e] - safe) * float(min(kBlock, p.Tk - kBlock * (t0 + r)))
                            : 0.f;
        sc[0][e] = w;
        wsum += w;
      }
      st.den = st.den * alpha + wsum;
      st.m = mnew;
#pragma unroll
      for (int dt = 0; dt < S::DT; ++dt) st.acc[dt] *= alpha;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bf16x8 bw = pack8(sc[0], 8 * c);
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt) {
          const uint16_t* row = vct + int64_t(dt * 32 + col) * p.NKBP + t0 + 16 * c + 4 * hh;
          const u32x2 lo = load8(row);
          const u32x2 hi = load8(row + 8);
          const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          st.acc[dt] = mfma32x32x16(as_bf16x8(a), bw, st.acc[dt]);
        }
      }
    }
  }

  // 5. Exact blocks through the LDS ring (this wave's key half).
  __syncthreads();  // Q staging is dead; the ring is free
  const uint16_t* head_tiles = p.tiles + head * p.NKB * S::TILE;
  MaskCursor cursor{s_mask, 0, s_mask[0]};
  exact_stream<D, NT, 1>(head_tiles, ring, nsel, cursor, p.Tk, p.scale_log2, kh, qf, wave, lane, st);

  // 6. Merge the key halves (waves 2, 3 -> waves 0, 1) and store.
  __syncthreads();
  float* scratch = reinterpret_cast<float*>(ring);  // [qh][value][lane], value = acc..., m, den
  constexpr int NV = S::DT * 16 + 2;
  if (kh == 1) {
    float* dst = scratch + qh * NV * kWave;
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) dst[(dt * 16 + e) * kWave + lane] = st.acc[dt][e];
    dst[(NV - 2) * kWave + lane] = st.m;
    dst[(NV - 1) * kWave + lane] = st.den;
  }
  __syncthreads();
  if (kh == 0) {
    const float* src = scratch + qh * NV * kWave;
    const float m1 = src[(NV - 2) * kWave + lane];
    const float d1 = src[(NV - 1) * kWave + lane];
    const float m = fmaxf(st.m, m1);
    const float safe = m == kNegInf ? 0.f : m;
    const float a0 = fast_exp2(st.m - safe), a1 = fast_exp2(m1 - safe);
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st.acc[dt][e] = st.acc[dt][e] * a0 + src[(dt * 16 + e) * kWave + lane] * a1;
    st.den = st.den * a0 + d1 * a1;
    store_output<D>(p, b, h, q0 + myq, hh, st);
  }
}

template <int D>
__global__ __launch_bounds__(256, 2) void dense_attention_kernel(AttnParams p) {
  using S = Shape<D>;
  constexpr int NT = 256;
  constexpr int QROWS = 128;
  constexpr int Q_ELEMS = QROWS * S::KS;
  constexpr int RING = 2 * S::TILE > Q_ELEMS ? 2 * S::TILE : Q_ELEMS;
  __shared__ __align__(16) uint16_t ring[RING];

  const int nq_tiles = (p.Tq + QROWS - 1) / QROWS;
  const TileTask task = xcd_task(blockIdx.x, nq_tiles);
  if (task.bh < 0) return;
  const int qt = task.tile;
  const int bh = task.bh;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int q0 = qt * QROWS;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, hh = lane >> 5;

  for (int idx = tid; idx < QROWS * S::DC; idx += NT) {
    const int r = idx / S::DC, c = idx % S::DC;
    const int t = q0 + r;
    const u32x4 x = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(ring + r * S::KS + 8 * c) = x;
  }
  __syncthreads();
  bf16x8 qf[S::KT];
  const int myq = 32 * wave + col;
#pragma unroll
  for (int ks = 0; ks < S::KT; ++ks)
    qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(ring + myq * S::KS + ks * 16 + 8 * hh));
  __syncthreads();

  State<D> st;
  state_init(st);
  exact_stream<D, NT, 2>(p.tiles + head * p.NKB * S::TILE, ring, p.NKB, RangeCursor{0}, p.Tk,
                         p.scale_log2, 0, qf, wave, lane, st);
  store_output<D>(p, b, h, q0 + myq, hh, st);
}

hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned grid = xcd_grid(p.B * p.H, p.NQB);
  if (D == 128)
    hipLaunchKernelGGL(sol_attention_kernel<128>, dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(sol_attention_kernel<64>, dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_dense(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned grid = xcd_grid(p.B * p.H, (p.Tq + 127) / 128);
  if (D == 128)
    hipLaunchKernelGGL(dense_attention_kernel<128>, dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(dense_attention_kernel<64>, dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
