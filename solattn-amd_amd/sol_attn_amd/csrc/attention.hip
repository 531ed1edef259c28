// Fused SOL routing + attention, and the dense flash-attention control, for gfx950.
//
// Replaces the reference's `_threshold` (src/sol_attn_amd/kernels.py:52-64),
// `_sol` (kernels.py:101-182) and `_dense` (kernels.py:67-98).
//
// SOL workgroup = G 64-query blocks of one (batch, head), paired at the
// stride the pairing pass chose (adjacent blocks without one), two waves per
// query block.  Wave w owns query block w >> 1 and its queries
// 32*(w&1) .. +31, over all 64 keys of every tile, with its own FP32
// online-softmax state.
//   1. Q tiles -> LDS -> register fragments (MFMA B operand of S^T = K Q^T)
//   2. FP32 query mean (torch cascade order) and the Eq.15 cutoff
//      c = Qc.mu + beta * sqrt(sum Qc^2 var)                    (kernels.py:58-63)
//   3. centroid pass: the NCT centroid tiles (64 BF16 block centroids each)
//      stream through an R-slot LDS ring fed by global_load_lds DMA.  From
//      each tile in LDS: routing proxy_j = Qc . Kc_j (= mean over the block's
//      rows of q_r . Kc_j), selected = proxy > c OR sink / local / plan
//      protection, into an LDS bitmask (kernels.py:129-143); then the
//      unselected blocks contribute w = exp2(s - m) * valid_len,
//      O^T += Vc^T bf16(w)^T                                    (kernels.py:145-158)
//   4. exact pass: the union over the group of the selected exact tiles
//      (64 tokens each), ascending, through the same ring; each wave consumes
//      the tiles its query block selected: S^T = K Q^T, online softmax,
//      O^T += V^T bf16(P)^T                                     (kernels.py:159-178)
//   5. O = acc / den, BF16 store, exact count                   (kernels.py:179-182)
// Every contribution shares the FP32 online-softmax state of its wave, in log2
// units; empty states use max 0 for the rescale (kernels.py:148-150).
// The dense control streams every exact tile, 128 queries per workgroup
// (4 waves x 32 queries, full 64-key tiles per wave).
#include <algorithm>

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

// SOL launches dispatch the first `front` query tiles of every (entry, head)
// ahead of the rest, head-interleaved.  With query sinks those tiles hold the
// sink query blocks, whose workgroups stream every key block and run several
// times longer than the others; in xcd_task order the last heads' ones would
// start late and set the kernel's end (2 x 4,096 tokens x 16 heads with
// 128-token sinks: 251 -> 163 us).  The remaining tiles keep the xcd_task map.
__device__ __forceinline__ TileTask sol_task(int i, int ntiles, int front, int heads) {
  const int nfront = front * heads;
  if (i < nfront) return TileTask{i % heads, i / heads};
  if (ntiles <= front) return TileTask{-1, 0};
  TileTask t = xcd_task(i - nfront, ntiles - front);
  t.tile += front;
  return t;
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
  static constexpr int TILE = 2 * kBlock * D;  // K + V^T tile elements per 64-wide tile
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

// Max / sum of a value over the lane pair (l, l ^ 32) that shares one query.
__device__ __forceinline__ float pair_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& s, int base) {
  u32x4 pb;
#pragma unroll
  for (int i = 0; i < 4; ++i) pb[i] = pack_bf16x2(s[base + 2 * i], s[base + 2 * i + 1]);
  return as_bf16x8(pb);
}

// Wave-uniform copy of a 64-bit value, in an SGPR pair.  readfirstlane
// returns a signed int: each half goes through uint32_t so that the low word
// is zero-extended, never sign-extended into the high word.
__device__ __forceinline__ uint64_t uniform64(uint64_t x) {
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(x)));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(x >> 32)));
  return (uint64_t(hi) << 32) | uint64_t(lo);
}

// 16-byte global -> LDS DMA per lane: lane l reads sbase + lane_bytes and its
// bytes land at LDS address m + 16 l; sbase and m are wave-uniform.  The base
// travels in an SGPR pair (global "saddr" form) and the per-lane part is a
// 32-bit offset, so a refill holds no 64-bit per-lane addresses in vector
// registers.  Issued as inline assembly so that the compiler does not drain
// the vector memory counter before every LDS read (it cannot tell the ring's
// buffers apart); completion is awaited explicitly with wait_vmcnt before the
// barrier.  M0 (the LDS base register of the DMA) is saved and restored
// around it.
__device__ __forceinline__ void dma16(uint64_t sbase, uint32_t lane_bytes, uint32_t m) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m), "v"(lane_bytes), "s"(sbase)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((SOL_LDS const void*)p));
}

// DMA of one K + V^T tile pair (contiguous in HBM) into an LDS buffer, in
// kRounds rounds of one 16-byte chunk per lane: round r moves the 1 KB piece
// of wave w at byte offset 16 (r NT + 64 w).  A refill can be issued whole,
// or a few rounds at a time between a wave's score MFMAs, so that the wave's
// in-order instruction stream does not stall on a burst of DMA issues.
// Every round must be issued exactly once per refill.  Rounds are
// unconditional (no branch splits the MFMA schedule): a stream with no
// further tile refills the slot with a tile it already read, into a slot no
// later tile uses.
template <int D, int NT>
struct TileRefill {
  static constexpr int kChunks = Shape<D>::TILE / 8;  // 16-byte chunks per tile pair
  static constexpr int kRounds = kChunks / NT;
  static_assert(kChunks % NT == 0, "tile pair must split evenly over the workgroup");
  uint64_t src;         // wave-uniform address of this wave's first chunk
  uint32_t lds;         // wave-uniform LDS address of the same chunk
  uint32_t lane_bytes;  // 16 * lane

  __device__ __forceinline__ TileRefill(const uint16_t* tile, uint32_t dst_lds, int wave, int lane)
      : src(uniform64(reinterpret_cast<uint64_t>(tile) + uint64_t(wave) * (kWave * 16))),
        lds(uint32_t(__builtin_amdgcn_readfirstlane(dst_lds + uint32_t(wave) * (kWave * 16)))),
        lane_bytes(uint32_t(lane) * 16u) {}

  __device__ __forceinline__ void round(int r) const {
    // The round's offset passes through an empty asm so that it is formed
    // here from an immediate, not kept live in registers of its own across
    // the whole stream.
    uint32_t off = uint32_t(r) * (NT * 16);
    asm volatile("" : "+s"(off));
    dma16(src + off, lane_bytes, lds + off);
  }
  __device__ __forceinline__ void all() const {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) round(r);
  }
  // The rounds that belong after step k of an N-step schedule.
  template <int N>
  __device__ __forceinline__ void after_step(int k) const {
#pragma unroll
    for (int r = k * kRounds / N; r < (k + 1) * kRounds / N; ++r) round(r);
  }
};

// A refill with nothing to load (single-slot ring).
struct NoRefill {
  __device__ __forceinline__ void all() const {}
  template <int N>
  __device__ __forceinline__ void after_step(int) const {}
};

template <int D, int NT>
__device__ __forceinline__ void tile_dma(const uint16_t* src, uint32_t dst_lds, int wave, int lane) {
  TileRefill<D, NT>(src, dst_lds, wave, lane).all();
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without a memory fence: LDS DMA completion is awaited
// explicitly with s_waitcnt vmcnt, so the in-flight prefetch of the next tile
// is not drained here.  The "memory" clobber keeps LDS accesses on their side.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Returns x through an empty asm statement.  Applied to a lane index inside a
// tile loop, it makes the addresses derived from it be formed per tile rather
// than hoisted out of the loop, where dozens of lane-dependent offsets would
// stay live (and spill) for the whole stream.
__device__ __forceinline__ int fresh(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Key row (inside a 64-row tile) of element e of this lane's 32-key half t:
// in the 32x32 MFMA result layout, lane half hh holds rows
// 8 (e / 4) + 4 hh + e % 4 of each 32-row half.
__device__ __forceinline__ int tile_row(int t, int e, int hh) {
  return 32 * t + 8 * (e >> 2) + 4 * hh + (e & 3);
}

// Lazy online softmax: the wave's running max m (log2 units) moves only when
// some query's max exceeds it by more than kRescaleSlack.  Otherwise the
// probabilities exp2(s c - m) may exceed 1 by up to 2^kRescaleSlack, which
// FP32 sums and BF16 products carry at unchanged relative precision; acc and
// den always share m, so O = acc / den is unaffected.  The common case has
// no data-dependent branch, so a half's softmax can be spread between
// matrix-core instructions.
constexpr float kRescaleSlack = 8.f;

// Materialises a value at this point of the instruction stream, so that the
// work producing it stays ahead of a following branch (where the scheduler
// can overlap it with matrix-core work) instead of being sunk past it.
template <typename T>
__device__ __forceinline__ void pin(T& x) {
  asm volatile("" : "+v"(x));
}

// Softmax of one 32-key half of raw scores s (absent keys -inf; c = scale *
// log2(e)), in 8 stages that a caller places between MFMAs: max; the
// wave-uniform rescale decision, new max and alpha; 4 x 4 probabilities
// exp2(s c - m); BF16 packing into pb[16-key c]; den update.  The caller
// multiplies acc by alpha when `rescale` is set.
template <int D>
struct HalfSoftmax {
  f32x16 s;
  float mx, alpha, neg_m, lsum;
  bool rescale;
  bf16x8 pb[2];

  __device__ __forceinline__ void stage(int k, State<D>& st, float c) {
    if (k == 0) {
      mx = kNegInf;
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[e]);
    } else if (k == 1) {
      mx = pair_max(mx) * c;
      rescale = __builtin_amdgcn_ballot_w64(mx > st.m + kRescaleSlack) != 0;
      const float mnew = rescale ? fmaxf(st.m, mx) : st.m;
      alpha = fast_exp2(st.m - (mnew == kNegInf ? 0.f : mnew));  // 1 without a rescale (0 before any key)
      st.m = mnew;
      neg_m = mnew == kNegInf ? 0.f : -mnew;
      lsum = 0.f;
    } else if (k < 6) {
#pragma unroll
      for (int e = 4 * (k - 2); e < 4 * (k - 1); ++e) {
        const float pe = fast_exp2(fmaf(s[e], c, neg_m));
        s[e] = pe;
        lsum += pe;
      }
    } else if (k == 6) {
      pb[0] = pack8(s, 0);
      pb[1] = pack8(s, 8);
      pin(pb[0]);
      pin(pb[1]);
    } else {
      st.den = st.den * alpha + lsum;
      pin(st.den);
    }
  }
  // Part k of n (n = 4 or 8) of the stages.
  template <int N>
  __device__ __forceinline__ void part(int k, State<D>& st, float c) {
#pragma unroll
    for (int i = k * 8 / N; i < (k + 1) * 8 / N; ++i) stage(i, st, c);
  }
};

// acc *= alpha, in place (the accumulator keeps its registers on both sides
// of the rare rescale branch instead of being copied).
template <int D>
__device__ __forceinline__ void rescale_acc(State<D>& st, float alpha) {
#pragma unroll
  for (int dt = 0; dt < Shape<D>::DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(st.acc[dt][e]) : "v"(alpha));
}

// This lane's element offsets of its MFMA operand reads inside a K + V^T
// tile pair (see TileLayout): K fragment (t, ks) at k_row + 32 t D +
// (k_x ^ 16 ks), V^T fragment (t, c4, dt) at kElems + v_row + 2048 dt +
// (v_x ^ (32 t + 16 c4)); the per-read parts are immediates or one XOR-add.
template <int D>
struct FragLane {
  int k_row, k_x, v_row, v_x;
  __device__ __forceinline__ FragLane(int col, int hh)
      : k_row(col * D),
        k_x(TileLayout<D>::k_lane_xor(col, hh)),
        v_row(TileLayout<D>::kElems + col * kBlock),
        v_x(TileLayout<D>::vt_lane_xor(col, hh)) {}
  __device__ __forceinline__ u32x4 k(const uint16_t* buf, int t, int ks) const {
    return *reinterpret_cast<const u32x4*>(buf + k_row + 32 * t * D + (k_x ^ (16 * ks)));
  }
  __device__ __forceinline__ u32x4 v(const uint16_t* buf, int t, int c4, int dt) const {
    return *reinterpret_cast<const u32x4*>(buf + v_row + 32 * kBlock * dt + (v_x ^ (32 * t + 16 * c4)));
  }
};

// Ends a scheduling chunk: nothing moves across it, so the hand-placed
// interleave of matrix-core, LDS, DMA and VALU work below is kept.
__device__ __forceinline__ void chunk_end() { __builtin_amdgcn_sched_barrier(0); }

// One 64-key tile, software-pipelined over its two 32-key halves inside the
// wave so that the VALU softmax work overlaps the MFMAs:
//   chunk 0        half 0's K reads
//   chunks 1..KT   half 0's score MFMAs; half 1's K reads
//   next KT        half 1's score MFMAs; half 0's softmax; half 0's V^T reads
//   [rescale]
//   next 2 DT      half 0's P V MFMAs; half 1's softmax; half 1's V^T reads
//   [rescale]      half 1's P V MFMAs
// The refill's DMA rounds are spread over the 2 KT score chunks.  Scores
// start from bias(t) when BIASED (-inf drops a key, log2(len) / c adds a
// centroid's ln(len) logit term), else from 0.
template <int D, bool BIASED, typename Bias, typename Refill>
__device__ __forceinline__ void tile_attend(State<D>& st, const uint16_t* buf,
                                            const bf16x8 (&qf)[Shape<D>::KT], int col, int hh, float c,
                                            Bias bias, const Refill& refill) {
  constexpr int KT = Shape<D>::KT, DT = Shape<D>::DT;
  static_assert(KT == 2 * DT, "score and P V chunk counts match");
  const FragLane<D> fl(fresh(col), fresh(hh));
  u32x4 k0[KT], k1[KT];
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) k0[ks] = fl.k(buf, 0, ks);
  HalfSoftmax<D> h0, h1;
  h0.s = BIASED ? bias(0) : zero16();
  chunk_end();
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) {
    h0.s = mfma32x32x16(as_bf16x8(k0[ks]), qf[ks], h0.s);
    k1[ks] = fl.k(buf, 1, ks);
    refill.template after_step<2 * KT>(ks);
    chunk_end();
  }
  u32x4 va[2][DT];
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) {
    if (ks == 0) h1.s = BIASED ? bias(1) : zero16();
    h1.s = mfma32x32x16(as_bf16x8(k1[ks]), qf[ks], h1.s);
    h0.template part<KT>(ks, st, c);
    if (ks >= KT / 2) {  // two of half 0's 2 DT = KT V^T fragments per chunk
#pragma unroll
      for (int f = 2 * (ks - KT / 2); f < 2 * (ks - KT / 2) + 2; ++f)
        va[f / DT][f % DT] = fl.v(buf, 0, f / DT, f % DT);
    }
    refill.template after_step<2 * KT>(KT + ks);
    chunk_end();
  }
  if (h0.rescale) rescale_acc<D>(st, h0.alpha);
  u32x4 vb[2][DT];
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(va[c4][dt]), h0.pb[c4], st.acc[dt]);
    vb[c4][dt] = fl.v(buf, 1, c4, dt);
    h1.template part<2 * DT>(f, st, c);
    chunk_end();
  }
  if (h1.rescale) rescale_acc<D>(st, h1.alpha);
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(vb[c4][dt]), h1.pb[c4], st.acc[dt]);
  }
}

struct NoBias {
  __device__ __forceinline__ f32x16 operator()(int) const { return zero16(); }
};

// A full exact block (every key present).
template <int D, typename Refill>
__device__ __forceinline__ void full_tile(State<D>& st, const uint16_t* buf,
                                          const bf16x8 (&qf)[Shape<D>::KT], int col, int hh, float c,
                                          const Refill& refill) {
  tile_attend<D, false>(st, buf, qf, col, hh, c, NoBias{}, refill);
}

// Exact block j: a full block, or the tail block whose keys at or past tk
// start at -inf.  Only a stream's last exact tile can be the tail block.
template <int D, typename Refill>
__device__ __forceinline__ void exact_tile(State<D>& st, const uint16_t* buf, int j, int tk,
                                           const bf16x8 (&qf)[Shape<D>::KT], int col, int hh, float c,
                                           const Refill& refill) {
  if ((j + 1) * kBlock <= tk) {
    full_tile<D>(st, buf, qf, col, hh, c, refill);
  } else {
    const int lane_keys = fresh(tk - j * kBlock - 4 * hh);  // keys from this lane's first row on
    tile_attend<D, true>(st, buf, qf, col, hh, c,
                         [&](int t) {
                           f32x16 bias;
#pragma unroll
                           for (int e = 0; e < 16; ++e)
                             bias[e] = tile_row(t, e, 0) < lane_keys ? 0.f : kNegInf;
                           return bias;
                         },
                         refill);
  }
}

// Centroid tile ct: the block centroids 64 ct + r whose bit r is set in
// `approx` contribute logit q . Kc_j + ln(len_j) and value Vc_j: their scores
// start at log2(len_j) / c (c = scale * log2(e)), the others at -inf.  Only
// the lane's share of the row index is formed at run time.
template <int D, typename Refill>
__device__ __forceinline__ void centroid_tile(State<D>& st, const uint16_t* buf, int ct, uint64_t approx,
                                              int tk, const bf16x8 (&qf)[Shape<D>::KT], int col, int hh,
                                              float c, const Refill& refill) {
  const uint64_t lane_approx = approx >> (4 * hh);
  const float inv_c = 1.f / c;
  // Every block of the tile is whole unless it holds the sequence's partial
  // last block; whole blocks share one offset, log2(64) / c, computed as the
  // per-block formula computes it at len 64.
  const bool whole_tile = kBlock * kBlock * (ct + 1) <= tk;
  const float whole = __builtin_amdgcn_logf(float(kBlock)) * inv_c;
  const int lane_tokens = tk - kBlock * (kBlock * ct + 4 * hh);  // keys from the lane's first block on
  tile_attend<D, true>(st, buf, qf, col, hh, c,
                       [&](int t) {
                         f32x16 bias;
                         if (whole_tile) {
#pragma unroll
                           for (int e = 0; e < 16; ++e)
                             bias[e] = ((lane_approx >> tile_row(t, e, 0)) & 1u) ? whole : kNegInf;
                         } else {
#pragma unroll
                           for (int e = 0; e < 16; ++e) {
                             const int row = tile_row(t, e, 0);
                             const int len = min(kBlock, lane_tokens - kBlock * row);
                             bias[e] = ((lane_approx >> row) & 1u)
                                           ? __builtin_amdgcn_logf(float(len)) * inv_c : kNegInf;
                           }
                         }
                         return bias;
                       },
                       refill);
}

template <int D>
__device__ __forceinline__ void store_output(const AttnParams& p, int b, int h, int t, int hh,
                                             const State<D>& st) {
  using S = Shape<D>;
  const float den = pair_sum(st.den);
  if (t >= p.Tq) return;
  int64_t row = int64_t(b) * p.Tq + t;
  if (p.out_index) {
    row = p.out_index[row];
    if (row < 0 || row >= p.out_rows) return;  // outside the output: not stored
  }
  uint16_t* orow = p.out + (row * p.H + h) * D;
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

// Waits until at most `ahead` tiles' DMA (the newest ones) are still in flight.
template <int kRounds>
__device__ __forceinline__ void wait_ahead(int ahead) {
  if (ahead >= 3) {
    wait_vmcnt<3 * kRounds>();
  } else if (ahead == 2) {
    wait_vmcnt<2 * kRounds>();
  } else if (ahead == 1) {
    wait_vmcnt<kRounds>();
  } else {
    wait_vmcnt<0>();
  }
}

// Barrier that publishes this workgroup's LDS accesses (no global-memory
// fence, so the ring's DMA in flight is not drained).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Streams `count` tiles through an R-slot LDS ring: while tile i is on the
// matrix cores, the DMA of tiles i+1 .. i+R-1 is in flight.  One barrier per
// tile: after it, tile i is visible to every wave and every wave has finished
// tile i-1, whose slot then receives tile i+R-1 (or, past the last tile, tile
// i again, read by nobody).  `runs` holds selected(id) and two consumers,
// hit(buf, id, refill) for the wave's tiles and miss(buf, id, refill) for
// the others; each consumes tile i and issues that refill's DMA rounds
// (between its score MFMAs, or all at once when it has nothing to compute).
// Consecutive tiles with the same selection run in an inner loop of their
// own, so the accumulator is not split across a per-tile branch.  The last
// tile goes to last(buf, id, refill) instead, so that the loop bodies hold
// only the common case (an exact stream's last tile may be a partial
// block).  `next()` yields tile references (ids, or tags that carry an
// id) in order; the tile each reference names is the same for every thread,
// while selected(ref) may differ between waves.  source(ref) is the tile's
// HBM address.  R = 1: one slot, refilled after a barrier (latency
// hidden by the other workgroups of the CU).  Two streams over the same ring
// are separated by a barrier.
// Selection predicate and the two tile consumers of a stream.
template <typename Sel, typename Hit, typename Miss>
struct TileRuns {
  Sel selected;
  Hit hit;
  Miss miss;
};

template <typename Sel, typename Hit, typename Miss>
__device__ __forceinline__ TileRuns<Sel, Hit, Miss> tile_runs(Sel selected, Hit hit, Miss miss) {
  return {selected, hit, miss};
}

template <int D, int NT, int R, typename Next, typename Source, typename Runs, typename Last>
__device__ __forceinline__ void tile_stream(uint16_t* ring, int count, Next next, Source source,
                                            Runs runs, Last last, int wave, int lane) {
  using S = Shape<D>;
  constexpr int kRounds = S::TILE / 8 / NT;
  static_assert(R >= 1 && R <= 4 && (R & (R - 1)) == 0, "ring depth 1, 2 or 4");
  static_assert(R < 2 || (R - 2) * kRounds <= 63, "vmcnt range");
  if (count <= 0) return;
  const uint32_t ring_lds = lds_address(ring);
  if constexpr (R == 1) {
    for (int i = 0; i < count; ++i) {
      const int id = next();
      TileRefill<D, NT>(source(id), ring_lds, wave, lane).all();
      wait_vmcnt<0>();
      ring_barrier();
      if (i + 1 < count) {
        if (runs.selected(id)) {
          runs.hit(ring, id, NoRefill{});
        } else {
          runs.miss(ring, id, NoRefill{});
        }
      } else {
        last(ring, id, NoRefill{});
      }
      lds_barrier();
    }
    return;
  }
  int ids[R > 1 ? R - 1 : 1];  // tiles i .. i+R-2 (uniform); shifted each iteration
#pragma unroll
  for (int s = 0; s < R - 1; ++s) {
    ids[s] = s < count ? next() : 0;
    if (s < count) tile_dma<D, NT>(source(ids[s]), ring_lds + uint32_t(s * S::TILE * 2), wave, lane);
  }
  auto step = [&](int i, auto&& fn) {
    wait_ahead<kRounds>(min(R - 2, count - 1 - i));
    lds_barrier();
    const int id = ids[0];
#pragma unroll
    for (int s = 0; s < R - 2; ++s) ids[s] = ids[s + 1];
    int idn = id;
    if (i + R - 1 < count) {
      idn = next();
      ids[R - 2] = idn;
    }
    fn(ring + (i & (R - 1)) * S::TILE, id,
       TileRefill<D, NT>(source(idn), ring_lds + uint32_t(((i + R - 1) & (R - 1)) * S::TILE * 2), wave, lane));
  };
  int i = 0;
  while (i < count - 1) {
    if (runs.selected(ids[0])) {
      do {
        step(i, runs.hit);
        ++i;
      } while (i < count - 1 && runs.selected(ids[0]));
    } else {
      do {
        step(i, runs.miss);
        ++i;
      } while (i < count - 1 && !runs.selected(ids[0]));
    }
  }
  step(count - 1, last);
  // The last refills were issued after the last wait: drain them before the
  // ring is reused or the workgroup exits.
  wait_vmcnt<0>();
}

// Approximated blocks of centroid tile ct for one query block: valid blocks
// whose routing bit is clear.
__device__ __forceinline__ uint64_t tile_approx(const uint32_t* mask, int ct, int nkb) {
  const int nvalid = min(64, nkb - 64 * ct);
  const uint64_t valid = nvalid == 64 ? ~0ull : ((1ull << nvalid) - 1ull);
  const uint64_t sel = uint64_t(mask[2 * ct]) | (uint64_t(mask[2 * ct + 1]) << 32);
  return valid & ~sel;
}

// Exact tiles of a SOL workgroup: the union of its G query blocks' selected
// blocks, ascending, as tags 2 j + (whether the calling wave's own query
// block selected j), so that the stream needs no LDS read per tile to tell
// the wave's tiles from its partners'.  The exact phase starts (word 0
// loaded) on the first call; the word scan never passes the last mask word
// and every id is below nkb, so the cursor yields valid tiles even if called
// more than count() times.
template <int G>
struct UnionCursor {
  const uint32_t* mask;  // [G][stride] routing bitmasks
  const uint32_t* mine;  // the calling wave's own row of mask
  int stride, nkb;
  int word = -1;
  uint32_t bits = 0u, own = 0u;

  __device__ __forceinline__ uint32_t union_word(int w) const {
    uint32_t u = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) u |= mask[g * stride + w];
    return u;
  }
  __device__ __forceinline__ int count() const {
    int n = 0;
    for (int w = 0; w < (nkb + 31) / 32; ++w) n += __builtin_popcount(union_word(w));
    return n;
  }
  __device__ __forceinline__ void load(int w) {
    word = w;
    bits = union_word(w);
    own = uint32_t(__builtin_amdgcn_readfirstlane(mine[w]));  // wave-uniform: the wave's own row
  }
  __device__ __forceinline__ int operator()() {
    const int last = (nkb + 31) / 32 - 1;
    if (word < 0) load(0);
    while (bits == 0 && word < last) load(word + 1);
    if (bits == 0) return 0;  // unreachable when called count() times
    const int b = __builtin_ctz(bits);
    const int j = word * 32 + b;
    bits &= bits - 1u;
    return j < nkb ? 2 * j + int((own >> b) & 1u) : 0;
  }
};

struct RangeCursor {
  int j;
  __device__ __forceinline__ int operator()() { return j++; }
};

}  // namespace


// Query block of slot s (= group index * G + member) when group members are
// query blocks `stride` apart: within each run of 2 * stride blocks, block i
// pairs with block i + stride; blocks past the last full run keep their slot.
// A bijection on [0, n); slots >= n stay >= n (no query block).
__device__ __forceinline__ int slot_block(int s, int n, int stride) {
  if (stride <= 0) return s;
  const int run = 2 * stride;
  if (s >= (n / run) * run) return s;
  const int w = s % run;
  return (s / run) * run + (w >> 1) + (w & 1) * stride;
}

// __launch_bounds__ second argument: minimum waves per SIMD.  Two waves per
// SIMD leave each wave 256 VGPRs: the exact path keeps the 64-register
// accumulator, 32 registers of Q fragments and 64 of K or V fragments live.
// The bound names 256 threads for both workgroup forms, so the one-block form
// (128 threads) is held to the same budget (with its own 128-thread bound the
// compiler moves values through AGPRs instead).
template <int D, int G, int R>
__global__ __launch_bounds__(256, 2) void sol_attention_kernel(AttnParams p) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  constexpr int NT = 128 * G;
  constexpr int kMaskWords = kMaxKeyBlocks / 32;
  static_assert(R * S::TILE >= G * kBlock * S::KS, "Q staging must fit in the ring");
  __shared__ __align__(16) uint16_t ring[R * S::TILE];  // Q staging, then the tile ring
  __shared__ float s_qm[G][D];
  __shared__ float s_red[G][4];
  __shared__ float s_cut[G];
  __shared__ uint32_t s_mask[G][kMaskWords];

  const int ntiles = (p.NQB + G - 1) / G;
  const TileTask task = sol_task(blockIdx.x, ntiles, min(p.q_sink_blocks, ntiles), p.B * p.H);
  if (task.bh < 0) return;
  const int bh = task.bh;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, hh = lane >> 5;
  const int qg = wave >> 1, qh = wave & 1;  // query block in the group, query half
  const int lt = tid & 127;                  // thread index inside the query block's 2 waves
  const int qb0 = task.tile * G;  // first slot of this group
  // Query-block pairing stride (any value is a valid pairing; see slot_block).
  const int stride = p.pair_stride ? min(p.pair_stride[bh], p.NQB) : 0;
  const int qb = slot_block(qb0 + qg, p.NQB, stride);
  const bool live = qb < p.NQB;
  const int tk = batch_tokens(p.klen, b, p.Tk);  // this entry's key tokens
  const int nkb = (tk + kBlock - 1) / kBlock;      // its key blocks (<= p.NKB, the buffer stride)
  const int nct = (nkb + kBlock - 1) / kBlock;     // its centroid tiles (<= p.NCT)
  const float scale_log2 = p.scale_log2;

  // 1. Q tiles -> LDS -> fragments.
  for (int idx = tid; idx < G * kBlock * S::DC; idx += NT) {
    const int r = idx / S::DC, c = idx % S::DC;
    const int t = slot_block(qb0 + r / kBlock, p.NQB, stride) * kBlock + r % kBlock;
    const u32x4 x = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(ring + r * S::KS + 8 * c) = x;
  }
  __syncthreads();
  bf16x8 qf[S::KT];
  const int myq = 32 * qh + col;  // query inside the block
  {
    const uint16_t* qrow = ring + (qg * kBlock + myq) * S::KS;
#pragma unroll
    for (int ks = 0; ks < S::KT; ++ks)
      qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(qrow + ks * 16 + 8 * hh));
  }

  // 2. Query mean and cutoff per query block (sums in torch's cascade order).
  if (p.force == 0) {
    const int qlen = live ? min(kBlock, p.Tq - qb * kBlock) : 1;
    if (lt < D) {
      float tot = 0.f;
      for (int c = 0; c < 4; ++c) {
        float sum = 0.f;
        for (int i = 0; i < 16; ++i) {
          const int r = 16 * c + i;
          if (r < qlen) sum = __fadd_rn(sum, bf16_bits_to_f32(ring[(qg * kBlock + r) * S::KS + lt]));
        }
        tot = __fadd_rn(tot, sum);
      }
      s_qm[qg][lt] = __fdiv_rn(tot, float(qlen));
    }
    __syncthreads();
    float a = 0.f, g = 0.f;
    if (lt < D) {
      const float qm = s_qm[qg][lt];
      a = qm * p.mean[head * D + lt];
      if (p.cov) {
        // Full covariance: this feature's term of Qc^T cov Qc.
        const float* row = p.cov + (head * D + lt) * D;
        float sq = 0.f;
        for (int e = 0; e < D; ++e) sq = fmaf(row[e], s_qm[qg][e], sq);
        g = qm * sq;
      } else {
        g = qm * qm * p.var[head * D + lt];
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      a += __shfl_xor(a, off);
      g += __shfl_xor(g, off);
    }
    if (lane == 0) {
      s_red[qg][qh] = a;
      s_red[qg][2 + qh] = g;
    }
    __syncthreads();
    if (tid < G) {
      const float quad = s_red[tid][2] + s_red[tid][3];  // the full quadratic form may round below 0
      s_cut[tid] = (s_red[tid][0] + s_red[tid][1]) + p.beta * sqrtf(p.cov ? fmaxf(quad, 0.f) : quad);
    }
  }
  __syncthreads();  // cutoffs published; Q staging is dead and the ring is free
  const int64_t dbg_row = ((int64_t(b) * p.NQB + qb) * p.H + h) * p.NKB;
  if (live && p.dbg_cutoff && lt == 0)
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb) * p.H + h] =
        p.force == 0 ? s_cut[qg] * p.scale : (p.force == 1 ? kNegInf : -kNegInf);

  State<D> st;
  state_init(st);
  if (p.force == 1) {
    // 3'. beta = -inf: every block exact, no centroid pass.
    const int nwords = (nkb + 31) / 32;
    for (int i = tid; i < G * nwords; i += NT) {
      const int g = i / nwords, w = i % nwords;
      const int nvalid = min(32, nkb - 32 * w);
      s_mask[g][w] = slot_block(qb0 + g, p.NQB, stride) < p.NQB
                         ? (nvalid == 32 ? ~0u : ((1u << nvalid) - 1u)) : 0u;
    }
    if (live && p.dbg_selected)
      for (int j = lt; j < nkb; j += 128) p.dbg_selected[dbg_row + j] = 1;
    __syncthreads();
  } else {
    // 3. Centroid pass.  Per tile: routing of the tile's 64 blocks for every
    // query block of the group -- wave w scores blocks 32 (w & 1) + (lane & 31)
    // of query block w >> 1 over feature half lane >> 5, the halves summed
    // across the lane pair -- into the LDS bitmask; a barrier publishes the
    // mask; then the approximated blocks' contributions.
    const uint16_t* ctiles = p.ctiles + head * p.NCT * S::TILE;
    auto process = [&](const uint16_t* buf, int ct, const auto& refill) {
      const int r = fresh(32 * qh + col);  // centroid row inside the tile
      const int j = kBlock * ct + r;
      bool sel = false;
      if (live && j < nkb) {
        if (p.force == 0) {
          const int c0 = fresh(hh) * (S::DC / 2);  // first 16-byte chunk of this lane's feature half
          float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < S::DC / 2; ++c) {
            const int cc = c0 + c;
            const u32x4 x = *reinterpret_cast<const u32x4*>(buf + TL::k_offset(r, cc));
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t w = x[e >> 1];
              part[e & 3] = fmaf(s_qm[qg][8 * cc + e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)),
                                 part[e & 3]);
            }
          }
          const float proxy = pair_sum((part[0] + part[1]) + (part[2] + part[3]));
          sel = proxy > s_cut[qg];
          if (p.dbg_proxy && hh == 0) p.dbg_proxy[dbg_row + j] = proxy * p.scale;
        }
        sel = sel || (p.local_blocks >= 0 && abs(j - qb) <= p.local_blocks) || j < p.kv_sink_blocks ||
              qb < p.q_sink_blocks;
        if (p.protection) sel = sel || p.protection[(int64_t(b) * p.NQB + qb) * p.NKB + j] != 0;
        if (p.dbg_selected && hh == 0) p.dbg_selected[dbg_row + j] = sel ? 1 : 0;
      }
      const uint64_t bal = __ballot(sel);
      if (lane == 0) s_mask[qg][2 * ct + qh] = uint32_t(bal);
      lds_barrier();  // publishes the mask words
      // Branch-free: a tile with no approximated block for this query block
      // (or a query block past the end) has every score at -inf and adds
      // nothing.
      const uint64_t approx = live ? tile_approx(s_mask[qg], ct, nkb) : 0ull;
      centroid_tile<D>(st, buf, ct, approx, tk, qf, col, hh, scale_log2, refill);
    };
    auto always = [](int) { return true; };
    tile_stream<D, NT, R>(ring, nct, RangeCursor{0},
                          [&](int ct) { return ctiles + int64_t(ct) * S::TILE; },
                          tile_runs(always, process, process), process, wave, lane);
    lds_barrier();  // every wave is done with the ring's centroid tiles
  }
  if (live && p.counts && lt == 0) {
    int nsel = 0;
    for (int w = 0; w < (nkb + 31) / 32; ++w) nsel += __builtin_popcount(s_mask[qg][w]);
    p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = nsel;
  }

  // 4. Exact pass over the union of the group's selected blocks.  Only the
  // stream's last tile can be the partial tail block.
  // Tile ids travel as tags 2 j + own-selection bit (UnionCursor).
  UnionCursor<G> cursor{&s_mask[0][0], s_mask[qg], kMaskWords, nkb};
  const int count = cursor.count();
  const uint16_t* tiles = p.tiles + head * p.NKB * S::TILE;
  auto selected = [](int tag) { return (tag & 1) != 0; };
  auto hit = [&](const uint16_t* buf, int, const auto& refill) {
    full_tile<D>(st, buf, qf, col, hh, scale_log2, refill);
  };
  auto miss = [&](const uint16_t*, int, const auto& refill) { refill.all(); };
  tile_stream<D, NT, R>(
      ring, count, cursor, [&](int tag) { return tiles + int64_t(tag >> 1) * S::TILE; },
      tile_runs(selected, hit, miss),
      [&](const uint16_t* buf, int tag, const auto& refill) {
        if (tag & 1) {
          exact_tile<D>(st, buf, tag >> 1, tk, qf, col, hh, scale_log2, refill);
        } else {
          refill.all();
        }
      },
      wave, lane);

  // 5. Normalise and store.
  if (live) store_output<D>(p, b, h, qb * kBlock + myq, hh, st);
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
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const int tk = p.Tk;
  const float scale_log2 = p.scale_log2;
  const uint16_t* tiles = p.tiles + head * p.NKB * S::TILE;
  auto always = [](int) { return true; };
  auto hit = [&](const uint16_t* buf, int, const auto& refill) {
    full_tile<D>(st, buf, qf, col, hh, scale_log2, refill);
  };
  tile_stream<D, NT, 2>(
      ring, p.NKB, RangeCursor{0}, [&](int j) { return tiles + int64_t(j) * S::TILE; },
      tile_runs(always, hit, hit),
      [&](const uint16_t* buf, int j, const auto& refill) {
        exact_tile<D>(st, buf, j, tk, qf, col, hh, scale_log2, refill);
      },
      wave, lane);
  store_output<D>(p, b, h, q0 + myq, hh, st);
}

// LDS ring depth of the SOL kernel.
constexpr int kSolRing = 2;
// Below this many two-block workgroups the launch leaves CUs idle (256 CUs x
// 2 workgroups): such launches run one query block per workgroup instead,
// which doubles the workgroups and has no union to stream.  Both forms give
// bit-identical results (a wave's tiles, their order and its softmax state
// do not depend on its partner).  AttnParams::workgroup_form 1 or 2 forces
// one form (tests run both).
constexpr int64_t kSmallLaunchGroups = 512;

template <int D, int G>
void launch_sol_group(const AttnParams& p, hipStream_t stream) {
  // Grid of sol_task: the sink-holding tiles of every head, then xcd_task's.
  const int ntiles = (p.NQB + G - 1) / G, front = std::min(p.q_sink_blocks, ntiles);
  const unsigned grid = unsigned(front) * unsigned(p.B * p.H) + xcd_grid(p.B * p.H, ntiles - front);
  hipLaunchKernelGGL((sol_attention_kernel<D, G, kSolRing>), dim3(grid), dim3(128 * G), 0, stream, p);
}

hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream) {
  int g = int64_t(p.B) * p.H * ((p.NQB + 1) / 2) < kSmallLaunchGroups ? 1 : 2;
  if (p.workgroup_form == 1 || p.workgroup_form == 2) g = p.workgroup_form;
  if (D == 128) {
    if (g == 1) launch_sol_group<128, 1>(p, stream); else launch_sol_group<128, 2>(p, stream);
  } else {
    if (g == 1) launch_sol_group<64, 1>(p, stream); else launch_sol_group<64, 2>(p, stream);
  }
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
