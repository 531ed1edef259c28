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

#include "attn_common.h"

namespace sol {

namespace {
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
// centroid's ln(len) logit term), else from 0.  LATE: the bias (0 or -inf
// only) is added once a half's products are done instead, which keeps it out
// of the registers live across the score chain; the same values (x + 0 is x
// for the nonzero-signed sums a chain from +0 gives, and -inf either way).
template <int D, bool BIASED, typename Bias, typename Refill, bool LATE = false>
__device__ __forceinline__ void tile_attend(State<D>& st, const uint16_t* buf,
                                            const bf16x8 (&qf)[Shape<D>::KT], int col, int hh, float c,
                                            Bias bias, const Refill& refill) {
  constexpr bool EARLY = BIASED && !LATE;
  auto late = [&](f32x16& x, int t) {
    if constexpr (LATE) {
      const f32x16 b = bias(t);
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = x[e] + b[e];
    }
  };
  constexpr int KT = Shape<D>::KT, DT = Shape<D>::DT;
  static_assert(KT == 2 * DT, "score and P V chunk counts match");
  const FragLane<D> fl(fresh(col), fresh(hh));
  const uint32_t vbase = fl.v_base(buf);
  u32x4 k0[KT], k1[KT];
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) k0[ks] = fl.k(buf, 0, ks);
  // The raw scores of half t again (FastHalf::resolve), from the tile still in LDS.
  auto raw = [&](int t) {
    const FragLane<D> fr(fresh(col), fresh(hh));
    f32x16 s = EARLY ? bias(t) : zero16();
#pragma unroll
    for (int ks = 0; ks < KT; ++ks) s = mfma32x32x16(as_bf16x8(fr.k(buf, t, ks)), qf[ks], s);
    late(s, t);
    return s;
  };
  FastHalf<D> h0, h1;
  h0.s = EARLY ? bias(0) : zero16();
  chunk_end();
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) {
    h0.s = mfma32x32x16(as_bf16x8(k0[ks]), qf[ks], h0.s);
    k1[ks] = fl.k(buf, 1, ks);
    refill.template after_step<2 * KT>(ks);
    chunk_end();
  }
  late(h0.s, 0);
  u32x4 va[2][DT];
#pragma unroll
  for (int ks = 0; ks < KT; ++ks) {
    if (ks == 0) h1.s = EARLY ? bias(1) : zero16();
    h1.s = mfma32x32x16(as_bf16x8(k1[ks]), qf[ks], h1.s);
    h0.template part<KT>(ks, st, c);
    if (ks >= KT / 2) {  // two of half 0's 2 DT = KT V^T fragments per chunk
#pragma unroll
      for (int f = 2 * (ks - KT / 2); f < 2 * (ks - KT / 2) + 2; ++f)
        va[f / DT][f % DT] = fl.v(vbase, 0, f / DT, f % DT);
    }
    refill.template after_step<2 * KT>(KT + ks);
    chunk_end();
  }
  h0.resolve(st, c, [&] { return raw(0); });
  late(h1.s, 1);
  u32x4 vb[2][DT];
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(va[c4][dt]), h0.pb(c4), st.acc[dt]);
    vb[c4][dt] = fl.v(vbase, 1, c4, dt);
    h1.template part<2 * DT>(f, st, c);
    chunk_end();
  }
  h1.resolve(st, c, [&] { return raw(1); });
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(vb[c4][dt]), h1.pb(c4), st.acc[dt]);
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

// The rows of the sequence's partial last block j that hold its tk - 64 j
// keys: [64 - len, 64) when the block was DMA'd from rows shifted back to the
// sequence's last 64 rows (SHIFTED), else [0, len) (zero-padded tiles).
// Returned relative to this lane's rows, as the bounds a <= tile_row(t, e, 0)
// < z of the present keys.
template <bool SHIFTED>
__device__ __forceinline__ int2 tail_rows(int j, int tk, int hh) {
  const int len = tk - j * kBlock;
  const int lo = SHIFTED ? kBlock - len : 0;
  return make_int2(fresh(lo - 4 * hh), fresh(lo + len - 4 * hh));
}

// Exact block j: a full block, or the partial last block, whose absent keys
// start at -inf.  Only a stream's last exact tile can be that block.
template <int D, bool SHIFTED, typename Refill>
__device__ __forceinline__ void exact_tile(State<D>& st, const uint16_t* buf, int j, int tk,
                                           const bf16x8 (&qf)[Shape<D>::KT], int col, int hh, float c,
                                           const Refill& refill) {
  if ((j + 1) * kBlock <= tk) {
    full_tile<D>(st, buf, qf, col, hh, c, refill);
  } else {
    const int2 present = tail_rows<SHIFTED>(j, tk, hh);
    const auto absent = [&](int t) {
      f32x16 bias;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = tile_row(t, e, 0);
        bias[e] = row >= present.x && row < present.y ? 0.f : kNegInf;
      }
      return bias;
    };
    tile_attend<D, true, decltype(absent), Refill, true>(st, buf, qf, col, hh, c, absent, refill);
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

// The quantised-QK experiment's exact tile: S^T = K8 Q8^T on the INT8 matrix
// cores (D / 32 products per 32-key half instead of D / 16), then the INT32
// scores converted to FP32 and scaled inside the softmax by c8 = c s_q s_k
// (the lane's query scale, the tile's key scale); absent keys of the tail
// block (TAIL) start at -inf.  The softmax (FastHalf, which re-forms a
// half's integer scores in the uncommon case) and O^T += V^T P^T are those of
// tile_attend, with the same in-wave interleave: half 0's products; half
// 1's products with half 0's softmax and V^T reads; half 0's P V with half
// 1's softmax; half 1's P V.  The refill's DMA rounds are spread over the
// 2 D / 32 score chunks.
template <int D, bool TAIL, typename Refill>
__device__ __forceinline__ void tile_attend_i8(State<D>& st, const uint16_t* buf, const i32x4 (&q8)[D / 32],
                                               int col, int hh, float c8, int2 present, const Refill& refill) {
  constexpr int K8 = D / 32, DT = Shape<D>::DT;
  static_assert(K8 == DT, "two V^T fragments of half 0 per score chunk");
  const FragLane<D> fl(fresh(col), fresh(hh));
  const uint32_t vbase = fl.v_base(buf);
  const int8_t* kbuf = reinterpret_cast<const int8_t*>(buf);
  const int c0 = fresh(col);
  const int krow = c0 * D;                                 // row col of the K8 tile
  const int kx = 16 * (fresh(hh) ^ K8Layout<D>::swizzle(c0));  // chunk 2 ks8 + hh at kx ^ 32 ks8
  auto kfrag = [&](int t, int ks8) {
    return *reinterpret_cast<const i32x4*>(kbuf + krow + 32 * t * D + (kx ^ (32 * ks8)));
  };
  auto to_scores = [&](const i32x16& x, int t) {
    f32x16 sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sc[e] = float(x[e]);
      if (TAIL && (tile_row(t, e, 0) < present.x || tile_row(t, e, 0) >= present.y)) sc[e] = kNegInf;
    }
    return sc;
  };
  i32x4 k0[K8], k1[K8];
#pragma unroll
  for (int ks = 0; ks < K8; ++ks) k0[ks] = kfrag(0, ks);
  // The scores of half t again (FastHalf::resolve), from the tile still in LDS.
  auto raw = [&](int t) {
    i32x16 x;
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = 0;
#pragma unroll
    for (int ks = 0; ks < K8; ++ks) x = mfma32x32x32i8(kfrag(t, ks), q8[ks], x);
    return to_scores(x, t);
  };
  FastHalf<D> h0, h1;
  i32x16 i0, i1;
#pragma unroll
  for (int e = 0; e < 16; ++e) i0[e] = i1[e] = 0;
  chunk_end();
#pragma unroll
  for (int ks = 0; ks < K8; ++ks) {
    i0 = mfma32x32x32i8(k0[ks], q8[ks], i0);
    k1[ks] = kfrag(1, ks);
    refill.template after_step<2 * K8>(ks);
    chunk_end();
  }
  u32x4 va[2][DT];
#pragma unroll
  for (int ks = 0; ks < K8; ++ks) {
    i1 = mfma32x32x32i8(k1[ks], q8[ks], i1);
    if (ks == 0) h0.s = to_scores(i0, 0);
    h0.template part<K8>(ks, st, c8);
#pragma unroll
    for (int f = 2 * ks; f < 2 * ks + 2; ++f) va[f / DT][f % DT] = fl.v(vbase, 0, f / DT, f % DT);
    refill.template after_step<2 * K8>(K8 + ks);
    chunk_end();
  }
  h0.resolve(st, c8, [&] { return raw(0); });
  u32x4 vb[2][DT];
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(va[c4][dt]), h0.pb(c4), st.acc[dt]);
    vb[c4][dt] = fl.v(vbase, 1, c4, dt);
    if (f == 0) h1.s = to_scores(i1, 1);
    h1.template part<2 * DT>(f, st, c8);
    chunk_end();
  }
  h1.resolve(st, c8, [&] { return raw(1); });
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) {
    const int c4 = f / DT, dt = f % DT;
    st.acc[dt] = mfma32x32x16(as_bf16x8(vb[c4][dt]), h1.pb(c4), st.acc[dt]);
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
// while selected(ref) may differ between waves.  make(ref, lds) returns the
// refill (TileRefill, Q8Refill) that DMAs tile ref into the LDS slot at lds.
// R = 1: one slot, refilled after a barrier (latency
// hidden by the other workgroups of the CU).  Two streams over the same ring
// are separated by a barrier.  prologue() runs once the first tiles' DMA is
// issued (or, for an empty stream, at once), before the first wait.
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

// Refill factory for BF16 tile pairs at HBM address source(ref).
template <int D, int NT, typename Source>
__device__ __forceinline__ auto bf16_refills(Source source, int wave, int lane) {
  return [=](int ref, uint32_t lds) { return TileRefill<D, NT>(source(ref), lds, wave, lane); };
}

// Refill factory of key block j's K + V tile pair for (entry b, head h):
// from the pooled tile pairs (KT: indexed windows, or fewer than 64 keys) or
// straight from the K / V rows.
template <int D, int NT, bool KT>
__device__ __forceinline__ auto kv_refills(const AttnParams& p, int b, int h, int wave, int lane) {
  if constexpr (KT) {
    const uint16_t* tiles = p.tiles + (int64_t(b) * p.H + h) * p.NKB * Shape<D>::TILE;
    return bf16_refills<D, NT>([=](int j) { return tiles + int64_t(j) * Shape<D>::TILE; }, wave, lane);
  } else {
    const KvRows<D, NT> rows = kv_rows<D, NT>(p, b, h, wave * kWave + lane);
    return [=](int j, uint32_t lds) { return RowRefill<D, NT>(rows, j, lds, wave); };
  }
}

struct NoPrologue {
  __device__ __forceinline__ void operator()() const {}
};

template <int D, int NT, int R, typename Next, typename Make, typename Runs, typename Last,
          typename Prologue = NoPrologue>
__device__ __forceinline__ void tile_stream(uint16_t* ring, int count, Next next, Make make,
                                            Runs runs, Last last, int wave, int lane,
                                            Prologue prologue = {}) {
  using S = Shape<D>;
  constexpr int kRounds = decltype(make(0, 0u))::kRounds;
  static_assert(R >= 1 && R <= 4 && (R & (R - 1)) == 0, "ring depth 1, 2 or 4");
  static_assert(R < 2 || (R - 2) * kRounds <= 63, "vmcnt range");
  if (count <= 0) {
    prologue();
    return;
  }
  const uint32_t ring_lds = lds_address(ring);
  if constexpr (R == 1) {
    for (int i = 0; i < count; ++i) {
      const int id = next();
      make(id, ring_lds).all();
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
    if (s < count) make(ids[s], ring_lds + uint32_t(s * S::TILE * 2)).all();
  }
  // Work that overlaps the first tiles' DMA (LDS reads outside the ring slots
  // the stream fills before its first barrier).
  prologue();
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
    fn(ring + (i & (R - 1)) * S::TILE, id, make(idn, ring_lds + uint32_t(((i + R - 1) & (R - 1)) * S::TILE * 2)));
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

// Exact tiles of a SOL workgroup: the union of its G query blocks' selected
// blocks among bits [lo, hi) of a segment's masks, ascending, as tags
// 2 j + (whether the calling wave's own query block selected j), so that the
// stream needs no LDS read per tile to tell the wave's tiles from its
// partners'.  Only mask words overlapping [lo, hi) are read, and only their
// bits inside it.  The exact phase starts (word lo / 32 loaded) on the first
// call; the word scan never passes the range's last word, so the cursor
// yields valid tiles even if called more than count() times.
template <int G>
struct UnionCursor {
  const uint32_t* mask;  // [G][stride] routing bitmasks of a key segment
  const uint32_t* mine;  // the calling wave's own row of mask
  int stride;            // mask row stride (words)
  int lo, hi;            // the streamed bits of the segment's masks
  int base;              // the segment's first key block (bit i is block base + i)
  int word = -1;
  uint32_t bits = 0u, own = 0u;

  __device__ __forceinline__ uint32_t union_word(int w) const {
    uint32_t u = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) u |= mask[g * stride + w];
    return u & uint32_t(bit_range64(lo - 32 * w, hi - 32 * w));
  }
  __device__ __forceinline__ int count() const {
    int n = 0;
    for (int w = lo / 32; w < (hi + 31) / 32; ++w) n += __builtin_popcount(union_word(w));
    return n;
  }
  __device__ __forceinline__ void load(int w) {
    word = w;
    bits = union_word(w);
    own = uint32_t(__builtin_amdgcn_readfirstlane(mine[w]));  // wave-uniform: the wave's own row
  }
  __device__ __forceinline__ int operator()() {
    const int last = (hi + 31) / 32 - 1;
    if (word < 0) load(lo / 32);
    while (bits == 0 && word < last) load(word + 1);
    if (bits == 0) return 2 * (base + lo);  // unreachable when called count() times
    const int b = __builtin_ctz(bits);
    const int j = word * 32 + b;  // < hi: union_word keeps only bits inside the range
    bits &= bits - 1u;
    return 2 * (base + j) + int((own >> b) & 1u);
  }
};

struct RangeCursor {
  int j;
  __device__ __forceinline__ int operator()() { return j++; }
};

// FP32 mean of a query block's qlen staged rows (LDS, row stride KS) at
// feature f, in torch's cascade order: four sequential 16-row sums folded in
// order (kernels.py:56).
template <int D>
__device__ __forceinline__ float query_mean(const uint16_t* rows, int qlen, int f) {
  float tot = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    // The chunk's 16 values are read first (every staged row exists), so the
    // reads overlap; the sum then takes the block's rows in order.
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = bf16_bits_to_f32(rows[(16 * c + i) * Shape<D>::KS + f]);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (16 * c + i < qlen) sum = __fadd_rn(sum, x[i]);
    tot = __fadd_rn(tot, sum);
  }
  return __fdiv_rn(tot, float(qlen));
}

// Key moments (kernels.py:30-49: mean and clamped population variance of
// the BF16 centroids) of one feature of one head for the cutoff stage, loaded
// before the query mean (load) and formed after it (finish), so the loads'
// latency hides behind the query mean.  Three sources:
// - the pooling pass's mean and variance (AttnParams::mean / var);
// - its chunk sums (AttnParams::ksum, folds_moments key sequences), folded
//   in moments_kernel's order: the whole 16-block chunks summed in turn from
//   0, the partial chunk's sum (or 0) added to that, then the two 256-block
//   levels (0 below 256 blocks), and the divisions by NKB;
// - the K centroids of centroid tile 0 (AttnParams::tile_moments, at most 16
//   key blocks), with the pooling kernel's one-chunk formula: the centroids
//   summed in turn from 0, their squares likewise, the divisions by NKB.
// Either way the same roundings in the same order as the pooling kernels,
// so the same bits.  Every load is unconditional (indices clamped into the
// buffers) so that they issue back to back.
template <int D>
struct KeyMoments {
  float x[2][16];  // chunk sums and sums of squares, or the centroids (x[0])
  float mu = 0.f, var = 0.f;

  __device__ __forceinline__ void load(const AttnParams& p, int64_t head, int f) {
    using TL = TileLayout<D>;
    if (p.ksum) {
      const int nch = (p.NKB + kPoolChunk - 1) / kPoolChunk;  // <= 16
      const float* base = p.ksum + head * nch * 2 * D + f;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int cc = min(c, nch - 1);
        x[0][c] = base[(2 * cc) * D];
        x[1][c] = base[(2 * cc + 1) * D];
      }
    } else if (p.tile_moments) {
      const uint16_t* kt = p.ctiles + head * p.NCT * 2 * TL::kElems;  // tile 0, its K half
#pragma unroll
      for (int r = 0; r < 16; ++r) x[0][r] = bf16_bits_to_f32(kt[TL::k_offset(r, f / 8) + f % 8]);
    } else {
      mu = p.mean[head * D + f];
      var = p.cov ? 0.f : p.var[head * D + f];
    }
  }

  __device__ __forceinline__ void finish(const AttnParams& p) {
    const float n = float(p.NKB);
    if (p.ksum) {
      const int full = p.NKB / kPoolChunk;  // <= 15
      const bool partial = full * kPoolChunk < p.NKB;
      float a[2] = {0.f, 0.f}, r[2] = {0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 16; ++c)
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          if (c < full) a[w] = __fadd_rn(a[w], x[w][c]);
          else if (c == full && partial) r[w] = x[w][c];
        }
      const float m = __fdiv_rn(__fadd_rn(__fadd_rn(__fadd_rn(r[0], a[0]), 0.f), 0.f), n);
      const float sq = __fdiv_rn(__fadd_rn(__fadd_rn(__fadd_rn(r[1], a[1]), 0.f), 0.f), n);
      const float v = __fsub_rn(sq, __fmul_rn(m, m));
      mu = m;
      var = v > 0.f ? v : 0.f;
    } else if (p.tile_moments) {
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (r < p.NKB) {
          s1 = __fadd_rn(s1, x[0][r]);
          s2 = __fadd_rn(s2, __fmul_rn(x[0][r], x[0][r]));
        }
      }
      const float m = __fdiv_rn(s1, n);
      const float v = __fsub_rn(__fdiv_rn(s2, n), __fmul_rn(m, m));
      mu = m;
      var = v > 0.f ? v : 0.f;
    }
  }
};

// The cutoff from the workgroup-summed terms: sum Qc mu + beta sqrt(the
// quadratic form), which the full covariance may round below 0
// (kernels.py:58-63).
__device__ __forceinline__ float cutoff_value(const AttnParams& p, float lin0, float lin1, float quad0,
                                              float quad1) {
  const float quad = quad0 + quad1;
  return (lin0 + lin1) + p.beta * sqrtf(p.cov ? fmaxf(quad, 0.f) : quad);
}

// Routing decision for key block j (row r of the centroid tile in LDS at
// buf) of query block qb in entry b: the proxy Qc . Kc_j over this lane's
// feature half (qm: the block's FP32 query mean), summed across the lane
// pair, above the cutoff -- or a key sink, local or plan-protected block
// (kernels.py:129-143).  Writes the diagnostics of row dbg_row.
template <int D>
__device__ __forceinline__ bool route_block(const AttnParams& p, const uint16_t* buf, const float* qm, float cut,
                                            int r, int j, int b, int qb, int hh, int64_t dbg_row) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  bool sel = false;
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
        part[e & 3] = fmaf(qm[8 * cc + e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)), part[e & 3]);
      }
    }
    const float proxy = pair_sum((part[0] + part[1]) + (part[2] + part[3]));
    sel = proxy > cut;
    if (p.dbg_proxy && hh == 0) p.dbg_proxy[dbg_row + j] = proxy * p.scale;
  }
  sel = sel || (p.local_blocks >= 0 && abs(j - qb) <= p.local_blocks) || j < p.kv_sink_blocks ||
        qb < p.q_sink_blocks;
  if (p.protection) sel = sel || p.protection[(int64_t(b) * p.NQB + qb) * p.NKB + j] != 0;
  if (p.dbg_selected && hh == 0) p.dbg_selected[dbg_row + j] = sel ? 1 : 0;
  return sel;
}

}  // namespace



// __launch_bounds__ second argument: minimum waves per SIMD.  Two waves per
// SIMD leave each wave 256 VGPRs: the exact path keeps the 64-register
// accumulator, 32 registers of Q fragments and 64 of K or V fragments live.
// The bound names 256 threads for both workgroup forms, so the one-block form
// (128 threads) is held to the same budget (with its own 128-thread bound the
// compiler moves values through AGPRs instead).
template <int D, int G, int R, bool Q8, bool KT, bool SEG>
__global__ __launch_bounds__(256, 2) void sol_attention_kernel(AttnParams p) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  constexpr int NT = 128 * G;
  constexpr int kMaskWords = kMaxKeyBlocks / 32;
  static_assert(R * S::TILE >= G * kBlock * S::KS, "Q staging must fit in the ring");
  __shared__ __align__(256) uint16_t ring[R * S::TILE];  // Q staging, then the tile ring
  __shared__ float s_qm[G][D];  // in-kernel routing: query means, partial sums, cutoffs
  __shared__ float s_red[G][4];
  __shared__ float s_cut[G];
  __shared__ uint32_t s_mask[G][kMaskWords];

  const int ntiles = (p.NQB + G - 1) / G;
  const int front = min(p.q_sink_blocks, ntiles);
  const int split_tiles = sink_split_tiles(p.splits, p.q_sink_blocks, G, front);
  TileTask task = sol_task(blockIdx.x, ntiles, front, split_tiles, p.B * p.H, p.splits);
  if (task.bh < 0) return;
  if (G == 2 && p.order && task.tile >= front)  // the order_kernel's deal of the regular tiles
    task.tile = front + p.order[int64_t(task.bh) * p.NQB + task.tile - front];
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
  const int stride = p.pair_stride && p.splits == 1 ? min(p.pair_stride[bh], p.NQB) : 0;
  const int qb = slot_block(qb0 + qg, p.NQB, stride);
  const bool live = qb < p.NQB;
  const int tk = batch_tokens(p.klen, b, p.Tk);  // this entry's key tokens
  const int nkb = (tk + kBlock - 1) / kBlock;      // its key blocks (<= p.NKB, the buffer stride)
  // A split front tile's workgroup routes and attends key blocks [range.x,
  // range.y) only and leaves its partial state to sol_merge_kernel.
  const int nsplit = task.tile < split_tiles ? p.splits : 1;
  const int2 range = split_range(task.split, nsplit, nkb);
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
  // Quantised-QK experiment: the query row as INT8 with one symmetric scale
  // s_q = max|q| / 127 (round to nearest even, clamped to +-127).  The lane
  // holds features 32 ks8 + 16 hh .. +15 of product ks8, as the K8 tile rows do.
  i32x4 q8[Q8 ? D / 32 : 1];
  float csq = 0.f;  // c s_q
  if constexpr (Q8) {
    const uint16_t* qrow = ring + (qg * kBlock + myq) * S::KS;
    u32x4 raw[D / 32][2];
    float amax = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        raw[ks][hf] = *reinterpret_cast<const u32x4*>(qrow + 32 * ks + 16 * hh + 8 * hf);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = raw[ks][hf][e >> 1];
          amax = fmaxf(amax, fabsf(bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu))));
        }
      }
    amax = pair_max(amax);
    const float inv = amax > 0.f ? __fdiv_rn(127.f, amax) : 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        uint32_t packed = 0;
#pragma unroll
        for (int bt = 0; bt < 4; ++bt) {
          const int e = 4 * wd + bt;  // feature 32 ks + 16 hh + e
          const uint32_t w = raw[ks][e >> 3][(e & 7) >> 1];
          const float x = bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu));
          const int qi = int(fminf(fmaxf(rintf(__fmul_rn(x, inv)), -127.f), 127.f));
          packed |= (uint32_t(qi) & 0xFFu) << (8 * bt);
        }
        q8[ks][wd] = int32_t(packed);
      }
    csq = p.scale_log2 * __fdiv_rn(amax, 127.f);
  }

  // 2. In-kernel routing (no routing masks given): query mean and cutoff per
  // query block (sums in torch's cascade order).
  const bool routed = p.mask != nullptr;  // decisions precomputed by route_kernel
  if (p.force == 0 && !routed) {
    const int qlen = live ? min(kBlock, p.Tq - qb * kBlock) : 1;
    KeyMoments<D> km;  // this thread's feature of the key moments, loads issued first
    if (lt < D) km.load(p, head, lt);
    if (lt < D) s_qm[qg][lt] = query_mean<D>(ring + qg * kBlock * S::KS, qlen, lt);
    __syncthreads();
    float a = 0.f, g = 0.f;
    if (lt < D) {
      km.finish(p);
      const float qm = s_qm[qg][lt];
      a = qm * km.mu;
      if (p.cov) {
        // Full covariance: this feature's term of Qc^T cov Qc.  cov is
        // symmetric bit for bit, so thread lt reads column lt (coalesced).
        const float* col = p.cov + int64_t(head) * D * D + lt;
        float sq = 0.f;
        for (int e = 0; e < D; ++e) sq = fmaf(col[e * D], s_qm[qg][e], sq);
        g = qm * sq;
      } else {
        g = qm * qm * km.var;
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
    if (tid < G) s_cut[tid] = cutoff_value(p, s_red[tid][0], s_red[tid][1], s_red[tid][2], s_red[tid][3]);
  }
  __syncthreads();  // cutoffs published; Q staging is dead and the ring is free
  const int64_t dbg_row = ((int64_t(b) * p.NQB + qb) * p.H + h) * p.NKB;
  // With precomputed routing, route_kernel wrote the cutoffs and decisions
  // and their diagnostics (every block exact at beta = -inf needs none).
  if (live && p.dbg_cutoff && lt == 0 && task.split == 0 && (!routed || p.force == 1))
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb) * p.H + h] =
        p.force == 0 ? s_cut[qg] * p.scale : (p.force == 1 ? kNegInf : -kNegInf);

  State<D> st;
  state_init(st);
  if (p.force == 1 && live && p.dbg_selected)
    for (int j = lt; j < nkb; j += 128) p.dbg_selected[dbg_row + j] = 1;
  int nsel = 0;  // this query block's selected blocks (kept by thread lt == 0)
  // Stages 3 and 4 run once per segment of up to kMaxKeyBlocks key blocks
  // (the LDS bitmask's capacity; segment s starts at block s kMaxKeyBlocks,
  // which is centroid tile s kMaxKeyBlocks / 64), carrying one softmax
  // state: the segment's centroid pass, then its exact pass.  SEG = false
  // (key sequences of at most kMaxKeyBlocks blocks) compiles to one segment.
  const int nseg = SEG ? (nkb + kMaxKeyBlocks - 1) / kMaxKeyBlocks : 1;
  for (int si = 0; si < nseg; ++si) {
    const int seg = si * kMaxKeyBlocks;                       // the segment's first key block
    const int snkb = SEG ? min(kMaxKeyBlocks, nkb - seg) : nkb;  // its key blocks
    const int ct0 = seg / kBlock;                             // its first centroid tile
    // This workgroup's blocks of the segment, as bits of its masks.
    const int r0 = max(seg, range.x) - seg, r1 = min(seg + snkb, range.y) - seg;
    if (seg > 0) lds_barrier();  // every wave is done with the last segment's mask and ring slots
    if (p.force == 1) {
      // 3'. beta = -inf: every block exact, no centroid pass.
      const int nwords = (snkb + 31) / 32;
      for (int i = tid; i < G * nwords; i += NT) {
        const int g = i / nwords, w = i % nwords;
        const int nvalid = min(32, snkb - 32 * w);
        s_mask[g][w] = slot_block(qb0 + g, p.NQB, stride) < p.NQB
                           ? (nvalid == 32 ? ~0u : ((1u << nvalid) - 1u)) : 0u;
      }
      __syncthreads();
    } else {
      // 3. Centroid pass over the segment's centroid tiles (the tiles holding
      // blocks [r0, r1)).  Routing decisions come from route_kernel's masks
      // (loaded into the LDS bitmask, bit j - seg, before the stream) or are
      // formed here, tile by tile.
      const uint16_t* ctiles = p.ctiles + head * p.NCT * S::TILE;
      auto always = [](int) { return true; };
      const int ct_lo = ct0 + r0 / kBlock;
      const int nct = r1 > r0 ? ct0 + (r1 - 1) / kBlock - ct_lo + 1 : 0;
      const auto crefill = bf16_refills<D, NT>([=](int ct) { return ctiles + int64_t(ct) * S::TILE; }, wave, lane);
      if (routed) {
        const int nwords = (snkb + 31) / 32;
        for (int i = tid; i < G * nwords; i += NT) {
          const int g = i / nwords, w = i % nwords;
          const int qbg = slot_block(qb0 + g, p.NQB, stride);
          s_mask[g][w] = qbg < p.NQB ? p.mask[((head * p.NQB) + qbg) * p.NW + seg / 32 + w] : 0u;
        }
        __syncthreads();
        auto process = [&](const uint16_t* buf, int ct, const auto& refill) {
          // Branch-free: a tile with no approximated block for this query
          // block (or a query block past the end) has every score at -inf and
          // adds nothing.
          const uint64_t approx = live ? tile_approx(s_mask[qg], ct - ct0, r0, r1) : 0ull;
          centroid_tile<D>(st, buf, ct, approx, tk, qf, col, hh, scale_log2, refill);
        };
        tile_stream<D, NT, R>(ring, nct, RangeCursor{ct_lo}, crefill, tile_runs(always, process, process), process,
                              wave, lane);
      } else {
        // Per tile: routing of the tile's 64 blocks for every query block of
        // the group -- wave w scores blocks 32 (w & 1) + (lane & 31) of query
        // block w >> 1 over feature half lane >> 5, the halves summed across
        // the lane pair -- into the LDS bitmask; a barrier publishes the mask;
        // then the approximated blocks' contributions.
        auto process = [&](const uint16_t* buf, int ct, const auto& refill) {
          const int r = fresh(32 * qh + col);  // centroid row inside the tile
          const int j = kBlock * ct + r;
          bool sel = false;
          if (live && j >= seg + r0 && j < seg + r1)
            sel = route_block<D>(p, buf, s_qm[qg], s_cut[qg], r, j, b, qb, hh, dbg_row);
          const uint64_t bal = __ballot(sel);
          if (lane == 0) s_mask[qg][2 * (ct - ct0) + qh] = uint32_t(bal);
          lds_barrier();  // publishes the mask words
          // Branch-free: a tile with no approximated block for this query block
          // (or a query block past the end) has every score at -inf and adds
          // nothing.
          const uint64_t approx = live ? tile_approx(s_mask[qg], ct - ct0, r0, r1) : 0ull;
          centroid_tile<D>(st, buf, ct, approx, tk, qf, col, hh, scale_log2, refill);
        };
        tile_stream<D, NT, R>(ring, nct, RangeCursor{ct_lo}, crefill, tile_runs(always, process, process), process,
                              wave, lane);
      }
      lds_barrier();  // every wave is done with the ring's centroid tiles
    }
    if (live && p.counts && lt == 0)
      for (int w = r0 / 32; w < (r1 + 31) / 32; ++w)
        nsel += __builtin_popcount(s_mask[qg][w] & uint32_t(bit_range64(r0 - 32 * w, r1 - 32 * w)));

    // 4. Exact pass over the union of the group's selected blocks of the
    // segment.  Only the last segment's last tile can be the partial tail
    // block.  Tile ids travel as tags 2 j + own-selection bit (UnionCursor).
    UnionCursor<G> cursor{&s_mask[0][0], s_mask[qg], kMaskWords, r0, r1, seg};
    const int count = cursor.count();
    const auto kv = kv_refills<D, NT, KT>(p, b, h, wave, lane);
    auto selected = [](int tag) { return (tag & 1) != 0; };
    auto miss = [&](const uint16_t*, int, const auto& refill) { refill.all(); };
    if constexpr (!Q8) {
      auto hit = [&](const uint16_t* buf, int, const auto& refill) {
        full_tile<D>(st, buf, qf, col, hh, scale_log2, refill);
      };
      tile_stream<D, NT, R>(
          ring, count, cursor, [=](int tag, uint32_t lds) { return kv(tag >> 1, lds); },
          tile_runs(selected, hit, miss),
          [&](const uint16_t* buf, int tag, const auto& refill) {
            if (tag & 1) {
              exact_tile<D, !KT>(st, buf, tag >> 1, tk, qf, col, hh, scale_log2, refill);
            } else {
              refill.all();
            }
          },
          wave, lane);
    } else {
      // Quantised QK: INT8 K tiles and their scales (the V tiles as in the
      // BF16 stream).
      const int8_t* k8 = p.k8 + head * p.NKB * K8Layout<D>::kBytes;
      const float* k8s = p.k8_scale + head * p.NKB;
      auto make = [=](int tag, uint32_t lds) {
        const int j = tag >> 1;
        return Q8Refill<D, NT, decltype(kv(0, 0u))>(k8 + int64_t(j) * K8Layout<D>::kBytes, lds, wave, lane,
                                                    kv(j, lds));
      };
      auto hit = [&](const uint16_t* buf, int tag, const auto& refill) {
        tile_attend_i8<D, false>(st, buf, q8, col, hh, csq * k8s[tag >> 1], int2{}, refill);
      };
      tile_stream<D, NT, R>(
          ring, count, cursor, make, tile_runs(selected, hit, miss),
          [&](const uint16_t* buf, int tag, const auto& refill) {
            if (tag & 1) {
              const int j = tag >> 1;
              const float c8 = csq * k8s[j];
              if ((j + 1) * kBlock <= tk)
                tile_attend_i8<D, false>(st, buf, q8, col, hh, c8, int2{}, refill);
              else
                tile_attend_i8<D, true>(st, buf, q8, col, hh, c8, tail_rows<!KT>(j, tk, hh), refill);
            } else {
              refill.all();
            }
          },
          wave, lane);
    }

  }  // segments
  if (nsplit > 1) {
    // Partial state of this key range: the record of row (tile, part,
    // query) holds acc (features in output order), m, the pair-summed
    // denominator and the query block's count of selected blocks.
    const float den = pair_sum(st.den);
    float* rec = p.partial +
                 (((int64_t(bh) * split_tiles + task.tile) * nsplit + task.split) * (G * kBlock) + qg * kBlock + myq) *
                     kPartialRow<D>;
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = st.acc[dt][4 * k4 + i];
        *reinterpret_cast<f32x4*>(rec + dt * 32 + 8 * k4 + 4 * hh) = x;
      }
    if (hh == 0) {
      f32x4 x;
      x[0] = st.m;
      x[1] = den;
      x[2] = float(nsel);  // thread lt == 0's (the query block's first row)
      x[3] = 0.f;
      *reinterpret_cast<f32x4*>(rec + D) = x;
    }
    return;
  }
  if (live && p.counts && lt == 0) p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = nsel;

  // 5. Normalise and store.
  if (live) store_output<D>(p, b, h, qb * kBlock + myq, hh, st);
}

// The exact tiles of key-split group `grp` of KS: positions grp, grp + KS,
// ... of the query block's selected blocks (UnionCursor<1> tags), one per
// stream step for every group; a group whose list ends first gets the
// cursor's (valid, unselected) padding tags for the remaining step.
template <int KS>
struct SplitCursor {
  UnionCursor<1> all;
  int grp;
  __device__ __forceinline__ int operator()() {
    int tag = 0;
#pragma unroll
    for (int g = 0; g < KS; ++g) {
      const int t = all();
      if (g == grp) tag = t;
    }
    return tag;
  }
};

// Small launches (one query block per workgroup, a few hundred workgroups at
// most): the queries' dependency chains, not the matrix cores, set the time
// -- a two-wave workgroup per query block leaves three of a CU's four SIMDs
// idle and exposes every load, barrier and accumulation latency of its tile
// chain (a query-sink block's chain is every key block).  Here KS groups of
// two waves share a query block: wave (grp, qh) owns queries 32 qh .. +31 of
// it, and group grp attends exact tiles grp, grp + KS, ... of its selected
// blocks through a two-slot ring of its own, every group stepping in the
// same workgroup barrier, so a chain of n tiles takes ceil(n / KS) steps.
// Group 0 routes and adds the centroid contributions (skipped for a tile
// with no approximated block); at the end every group publishes its
// online-softmax state in LDS and merges and stores a share of the output
// features (m = max m_g, acc and den weighted by 2^(m_g - m), groups in
// order).  Decisions, counts and diagnostics are the
// one-block kernel's; the output agrees with it to rounding (other partial
// sums).  POOL (plain K / V rows, at most one pooling chunk of key blocks,
// no centroid tiles given): every workgroup forms its head's block centroids
// and diagonal moments in LDS in the pooling kernel's order and arithmetic
// (bit-identical values), so the whole call is this one launch.  Finite and
// +inf beta only (beta = -inf launches take sol_attention_kernel).
// The ring takes ~130 KB of LDS: one workgroup per CU, KS / 2 waves per SIMD.
template <int D, int KS, bool KT, bool POOL>
__global__ __launch_bounds__(128 * KS, KS / 2) void sol_small_kernel(AttnParams p) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  constexpr int NT = 128 * KS;
  constexpr int kMaskWords = kMaxKeyBlocks / 32;
  constexpr int NC = S::DT * 4;            // 4-feature output chunks per lane
  constexpr int kStateFloats = 4 * NC + 2;  // per lane: acc, m, den
  constexpr int QPT = kBlock * S::DC / NT;  // Q staging chunks per thread
  static_assert(!POOL || !KT, "in-kernel pooling reads plain K / V rows");
  static_assert(QPT * NT == kBlock * S::DC, "Q rows split evenly over the workgroup");
  static_assert(KS * 2 * kWave * kStateFloats * 4 <= 2 * KS * S::TILE * 2, "merge records fit the ring");
  // Group g's ring slots at 2 g TILE (the centroid pass streams through the
  // first two); Q staging and the pooled centroid tile alias them early on.
  __shared__ __align__(256) uint16_t ring[2 * KS * S::TILE];
  __shared__ float s_qm[D];
  __shared__ float s_red[4];
  __shared__ float s_mom[2][POOL ? D : 1];  // pooled key mean, variance
  __shared__ uint32_t s_mask[kMaskWords];

  const int nbh = p.B * p.H;
  const int bh = blockIdx.x % nbh, qb = blockIdx.x / nbh;  // every head's first blocks dispatch first
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 1, qh = wave & 1;
  const int col = lane & 31, hh = lane >> 5;
  const int myq = 32 * qh + col;
  const int tk = batch_tokens(p.klen, b, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  const int qlen = min(kBlock, p.Tq - qb * kBlock);
  const float scale_log2 = p.scale_log2;
  const bool routed = p.mask != nullptr;
  uint16_t* const ctile = ring + S::TILE;  // the pooled centroid tile (slot 1)

  // 1. Q rows -> LDS (slot 0) -> fragments; with POOL, the head's centroids
  // -> slot 1 in the tile layout (rows past the last block zero).  Every
  // global load is issued before the first LDS store that waits on one.
  u32x4 qx[QPT];
#pragma unroll
  for (int i = 0; i < QPT; ++i) {
    const int idx = tid + i * NT, r = idx / S::DC, c = idx % S::DC;
    const int t = qb * kBlock + r;
    qx[i] = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
  }
  auto stage_q = [&] {
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int idx = tid + i * NT, r = idx / S::DC, c = idx % S::DC;
      *reinterpret_cast<u32x4*>(ring + r * S::KS + 8 * c) = qx[i];
    }
  };
  // Pooling units: block jb of K (u < 16) or of V (u - 16), 16 rows x 16
  // bytes per lane, summed as the pooling kernel sums them.
  constexpr int DC = D / 8;
  constexpr int LPB = DC * 4;       // lanes per key block: 4 row quarters x DC chunks
  constexpr int BPI = kWave / LPB;  // blocks per wave and pass
  constexpr int PER_PASS = 2 * KS * BPI;
  constexpr int NU = 2 * kPoolChunk / PER_PASS;  // units per lane
  // One K and one V unit per lane: V's centroids are finished while the
  // workgroup routes, so its loads stay in flight through the cutoff.
  constexpr bool kLateV = POOL && NU == 2;
  static_assert(!POOL || NU % 2 == 0, "K and V blocks split evenly over the passes");
  const int sub = lane / LPB, r4 = (lane % LPB) / DC, dc = lane % DC;
  auto load_unit = [&](int u, u32x4 (&x)[16]) {
    const int jb = u % kPoolChunk;
    const int len = jb < nkb ? min(kBlock, tk - kBlock * jb) : 0;
    if (len > 0)
      load_rows16<16>(u >= kPoolChunk ? p.v : p.k, b, kBlock * jb + 16 * r4, kBlock * jb + len - 1, h, 8 * dc, x);
    return len;
  };
  auto finish_unit = [&](int u, const u32x4 (&x)[16], int len) {
    float sm[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sm[e] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (16 * r4 + i < len) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = x[i][e >> 1];
          sm[e] = __fadd_rn(sm[e], bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)));
        }
      }
    }
    float t1[8], t2[8], t3[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      t1[e] = __shfl(sm[e], lane + DC);
      t2[e] = __shfl(sm[e], lane + 2 * DC);
      t3[e] = __shfl(sm[e], lane + 3 * DC);
    }
    if (r4 == 0) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float m0 = 0.f, m1 = 0.f;
        if (len > 0) {
          m0 = __fdiv_rn(__fadd_rn(__fadd_rn(__fadd_rn(sm[e], t1[e]), t2[e]), t3[e]), float(len));
          m1 = __fdiv_rn(__fadd_rn(__fadd_rn(__fadd_rn(sm[e + 1], t1[e + 1]), t2[e + 1]), t3[e + 1]), float(len));
        }
        o[e >> 1] = pack_bf16x2(m0, m1);
      }
      const int jb = u % kPoolChunk;
      *reinterpret_cast<u32x4*>(ctile + (u >= kPoolChunk ? TL::kElems + TL::v_offset(jb, dc) : TL::k_offset(jb, dc))) = o;
    }
  };
  const int u_first = wave * BPI + sub;
  u32x4 xv[kLateV ? 16 : 1];
  int len_v = 0;
  if constexpr (POOL) {
    if constexpr (kLateV) {
      u32x4 xk[16];
      const int len_k = load_unit(u_first, xk);
      len_v = load_unit(u_first + PER_PASS, xv);
      stage_q();
      finish_unit(u_first, xk, len_k);
    } else {
      // Two units per lane in flight at once.
#pragma unroll 1
      for (int u0 = 0; u0 < 2 * kPoolChunk; u0 += 2 * PER_PASS) {
        const int ua = u0 + u_first, ub = ua + PER_PASS;
        u32x4 xa[16], xb[16];
        const int la = load_unit(ua, xa);
        const int lb = load_unit(ub, xb);
        if (u0 == 0) stage_q();
        finish_unit(ua, xa, la);
        finish_unit(ub, xb, lb);
      }
    }
    // Rows kPoolChunk .. 63 of both tiles are zero.
    for (int idx = tid; idx < 2 * (kBlock - kPoolChunk) * DC; idx += NT) {
      const int kv = idx / ((kBlock - kPoolChunk) * DC), rest = idx % ((kBlock - kPoolChunk) * DC);
      const int r = kPoolChunk + rest / DC, c = rest % DC;
      *reinterpret_cast<u32x4*>(ctile + (kv ? TL::kElems + TL::v_offset(r, c) : TL::k_offset(r, c))) = zero_u32x4();
    }
  } else {
    stage_q();
  }
  __syncthreads();
  bf16x8 qf[S::KT];
  {
    const uint16_t* qrow = ring + myq * S::KS;
#pragma unroll
    for (int ks = 0; ks < S::KT; ++ks)
      qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(qrow + ks * 16 + 8 * hh));
  }
  if constexpr (POOL) {
    // Diagonal moments of the BF16 centroids: sequential sums over the
    // blocks, E[x^2] - mu^2 clamped at 0, each step rounded on its own.
    if (tid < D) {
      float s1 = 0.f, s2 = 0.f;
      for (int jb = 0; jb < nkb; ++jb) {
        const float x = bf16_bits_to_f32(ctile[TL::k_offset(jb, tid / 8) + tid % 8]);
        s1 = __fadd_rn(s1, x);
        s2 = __fadd_rn(s2, __fmul_rn(x, x));
      }
      const float n = float(nkb);
      const float m = __fdiv_rn(s1, n);
      const float v = __fsub_rn(__fdiv_rn(s2, n), __fmul_rn(m, m));
      s_mom[0][tid] = m;
      s_mom[1][tid] = v > 0.f ? v : 0.f;
    }
  }

  // 2. In-kernel routing: query mean and cutoff (group 0's threads sum; every
  // thread forms the cutoff from the published sums).
  float cut = 0.f;
  if (p.force == 0 && !routed) {
    KeyMoments<D> km;  // this thread's feature of the key moments (pooled here: below)
    if (!POOL && tid < D) km.load(p, head, tid);
    if (tid < D) s_qm[tid] = query_mean<D>(ring, qlen, tid);
    __syncthreads();  // also: every read of the Q staging rows is done
    float a = 0.f, g = 0.f;
    if (tid < D) {
      const float qm = s_qm[tid];
      float mu;
      if (POOL) {
        mu = s_mom[0][tid];
      } else {
        km.finish(p);
        mu = km.mu;
      }
      a = qm * mu;
      if (p.cov) {
        const float* col = p.cov + int64_t(head) * D * D + tid;  // symmetric: column tid
        float sq = 0.f;
        for (int e = 0; e < D; ++e) sq = fmaf(col[e * D], s_qm[e], sq);
        g = qm * sq;
      } else {
        g = qm * qm * (POOL ? s_mom[1][tid] : km.var);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      a += __shfl_xor(a, off);
      g += __shfl_xor(g, off);
    }
    if (wave < 2 && lane == 0) {
      s_red[wave] = a;
      s_red[2 + wave] = g;
    }
    __syncthreads();
    cut = cutoff_value(p, s_red[0], s_red[1], s_red[2], s_red[3]);
  } else {
    __syncthreads();  // every wave's Q fragments are read: the ring is free
  }
  const int64_t dbg_row = ((int64_t(b) * p.NQB + qb) * p.H + h) * p.NKB;
  if (p.dbg_cutoff && tid == 0 && !routed)
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb) * p.H + h] = p.force == 0 ? cut * p.scale : -kNegInf;

  State<D> st;
  state_init(st);
  const int nwords = (nkb + 31) / 32;
  {
    // 3. Centroid pass (group 0 attends; every wave takes part in the
    // barriers and the ring's DMA).  Launches at beta = -inf take
    // sol_attention_kernel.
    if (routed) {
      for (int w = tid; w < nwords; w += NT) s_mask[w] = p.mask[(head * p.NQB + qb) * p.NW + w];
      __syncthreads();
    }
    if constexpr (POOL) {
      // The one centroid tile sits in slot 1: route from it now (and finish
      // its V rows); its contributions run in the exact stream's prologue,
      // over the first exact tiles' DMA (group 0's first slot is slot 0).
      if (!routed && grp == 0) {
        const int j = fresh(myq);
        const bool sel = j < nkb && route_block<D>(p, ctile, s_qm, cut, j, j, b, qb, hh, dbg_row);
        const uint64_t bal = __ballot(sel);
        if (lane == 0) s_mask[qh] = uint32_t(bal);
      }
      if constexpr (kLateV) finish_unit(u_first + PER_PASS, xv, len_v);
      lds_barrier();  // publishes the mask words and the V centroids
    } else {
      auto process = [&](const uint16_t* buf, int ct, const auto& refill) {
        if (!routed) {
          if (grp == 0) {
            const int r = fresh(myq);  // centroid row inside the tile
            const int j = kBlock * ct + r;
            const bool sel = j < nkb && route_block<D>(p, buf, s_qm, cut, r, j, b, qb, hh, dbg_row);
            const uint64_t bal = __ballot(sel);
            if (lane == 0) s_mask[2 * ct + qh] = uint32_t(bal);
          }
          lds_barrier();  // publishes the mask words
        }
        // The workgroup's one query block decides for every wave: a tile
        // without approximated blocks (a query-sink block's) is skipped.
        const uint64_t approx = tile_approx(s_mask, ct, 0, nkb);
        if (grp == 0 && approx != 0ull) {
          centroid_tile<D>(st, buf, ct, approx, tk, qf, col, hh, scale_log2, refill);
        } else {
          refill.all();
        }
      };
      const uint16_t* ctiles = p.ctiles + head * p.NCT * S::TILE;
      auto always = [](int) { return true; };
      const auto crefill = bf16_refills<D, NT>([=](int ct) { return ctiles + int64_t(ct) * S::TILE; }, wave, lane);
      tile_stream<D, NT, 2>(ring, (nkb + kBlock - 1) / kBlock, RangeCursor{0}, crefill,
                            tile_runs(always, process, process), process, wave, lane);
      lds_barrier();  // the ring's centroid tiles and the masks are settled
    }
  }
  int nsel = 0;
  if (p.counts && tid == 0)
    for (int w = 0; w < nwords; ++w) nsel += __builtin_popcount(s_mask[w] & uint32_t(bit_range64(0, nkb - 32 * w)));

  // 4. Exact pass: group grp's share of the selected blocks, ascending.
  {
    UnionCursor<1> all{s_mask, s_mask, kMaskWords, 0, nkb, 0};
    const int steps = (all.count() + KS - 1) / KS;
    const int wg = wave & 1;  // the wave inside its group
    const auto kv = kv_refills<D, 128, KT>(p, b, h, wg, lane);
    auto selected = [](int tag) { return (tag & 1) != 0; };
    auto hit = [&](const uint16_t* buf, int, const auto& refill) {
      full_tile<D>(st, buf, qf, col, hh, scale_log2, refill);
    };
    auto miss = [&](const uint16_t*, int, const auto& refill) { refill.all(); };
    tile_stream<D, 128, 2>(
        ring + grp * 2 * S::TILE, steps, SplitCursor<KS>{all, grp},
        [=](int tag, uint32_t lds) { return kv(tag >> 1, lds); }, tile_runs(selected, hit, miss),
        [&](const uint16_t* buf, int tag, const auto& refill) {
          if (tag & 1) {
            exact_tile<D, !KT>(st, buf, tag >> 1, tk, qf, col, hh, scale_log2, refill);
          } else {
            refill.all();
          }
        },
        wg, lane, [&] {
          if constexpr (POOL) {
            const uint64_t approx = tile_approx(s_mask, 0, 0, nkb);
            if (grp == 0 && approx != 0ull)
              centroid_tile<D>(st, ctile, 0, approx, tk, qf, col, hh, scale_log2, NoRefill{});
          }
        });
  }

  // 5. Merge and store, spread over the groups: every group publishes its
  // state; group g then combines output chunks c = g, g + KS, ... of every
  // state -- O = sum_s 2^(m_s - m) acc_s / sum_s 2^(m_s - m) den_s, m =
  // max_s m_s, states in order -- and stores them (store_output's rows).
  __syncthreads();  // every group's stream is done with the ring
  float* rec = reinterpret_cast<float*>(ring);
  auto state = [&](int g) { return rec + (g * 2 + qh) * (kWave * kStateFloats); };
  {
    float* mine = state(grp);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = st.acc[c / 4][4 * (c % 4) + i];
      *reinterpret_cast<f32x4*>(mine + (c * kWave + lane) * 4) = x;
    }
    mine[4 * NC * kWave + lane] = st.m;
    mine[4 * NC * kWave + kWave + lane] = st.den;
  }
  __syncthreads();
  float ms[KS], m = kNegInf;
#pragma unroll
  for (int g = 0; g < KS; ++g) {
    ms[g] = state(g)[4 * NC * kWave + lane];
    m = fmaxf(m, ms[g]);
  }
  float w[KS], den = 0.f;
#pragma unroll
  for (int g = 0; g < KS; ++g) {
    w[g] = ms[g] == kNegInf ? 0.f : fast_exp2(ms[g] - m);
    den = den + w[g] * state(g)[4 * NC * kWave + kWave + lane];
  }
  den = pair_sum(den);
  if (p.counts && tid == 0) p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = nsel;
  const int t = qb * kBlock + myq;
  if (t >= p.Tq) return;
  int64_t row = int64_t(b) * p.Tq + t;
  if (p.out_index) {
    row = p.out_index[row];
    if (row < 0 || row >= p.out_rows) return;  // outside the output: not stored
  }
  uint16_t* orow = p.out + (row * p.H + h) * D;
#pragma unroll
  for (int c = grp; c < NC; c += KS) {
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < KS; ++g) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(state(g) + (c * kWave + lane) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = o[i] + w[g] * x[i];
    }
    u32x2 v;
    v[0] = pack_bf16x2(__fdiv_rn(o[0], den), __fdiv_rn(o[1], den));
    v[1] = pack_bf16x2(__fdiv_rn(o[2], den), __fdiv_rn(o[3], den));
    *reinterpret_cast<u32x2*>(orow + (c / 4) * 32 + 8 * (c % 4) + 4 * hh) = v;
  }
}

template <int D, bool KT>
__global__ __launch_bounds__(256, 2) void dense_attention_kernel(AttnParams p) {
  using S = Shape<D>;
  constexpr int NT = 256;
  constexpr int QROWS = 128;
  constexpr int Q_ELEMS = QROWS * S::KS;
  constexpr int RING = 2 * S::TILE > Q_ELEMS ? 2 * S::TILE : Q_ELEMS;
  __shared__ __align__(256) uint16_t ring[RING];

  const int nq_tiles = (p.Tq + QROWS - 1) / QROWS;
  const TileTask task = balanced_task(blockIdx.x, 0, p.B * p.H, nq_tiles);
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
  auto always = [](int) { return true; };
  auto hit = [&](const uint16_t* buf, int, const auto& refill) {
    full_tile<D>(st, buf, qf, col, hh, scale_log2, refill);
  };
  tile_stream<D, NT, 2>(
      ring, p.NKB, RangeCursor{0}, kv_refills<D, NT, KT>(p, b, h, wave, lane), tile_runs(always, hit, hit),
      [&](const uint16_t* buf, int j, const auto& refill) {
        exact_tile<D, !KT>(st, buf, j, tk, qf, col, hh, scale_log2, refill);
      },
      wave, lane);
  store_output<D>(p, b, h, q0 + myq, hh, st);
}

// Combines the partial states of split sink tiles (sol_task): per query
// row, m = max_s m_s, O = sum_s 2^(m_s - m) acc_s / sum_s 2^(m_s - m) den_s
// over the parts in ascending order; stores O as store_output does, and the
// query block's count (the parts' counts summed).  One thread per row and 4
// features; rows [B H][split_tiles][G 64] (adjacent pairing: tile t holds
// query blocks G t ..).
constexpr int kMergeThreads = 256;

template <int D, int G>
__global__ __launch_bounds__(kMergeThreads) void sol_merge_kernel(AttnParams p, int split_tiles) {
  constexpr int kChunks = D / 4;
  constexpr int kRows = kMergeThreads / kChunks;
  constexpr int RW = kPartialRow<D>;
  constexpr int kTileRows = G * kBlock;
  const int nsplit = p.splits;
  const int64_t row = int64_t(blockIdx.x) * kRows + threadIdx.x / kChunks;
  const int c = threadIdx.x % kChunks;
  if (row >= int64_t(p.B) * p.H * split_tiles * kTileRows) return;
  const int r = int(row % kTileRows);   // qg 64 + query
  const int64_t bt = row / kTileRows;   // bh split_tiles + tile
  const int tile = int(bt % split_tiles), bh = int(bt / split_tiles);
  const int h = bh % p.H, b = bh / p.H;
  const int qb = tile * G + r / kBlock;
  if (qb >= p.NQB) return;
  const float* rec0 = p.partial + (bt * nsplit * kTileRows + r) * RW;
  const int64_t part = int64_t(kTileRows) * RW;  // floats between one row's parts
  float m = kNegInf;
  for (int s = 0; s < nsplit; ++s) m = fmaxf(m, rec0[s * part + D]);
  float den = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  int count = 0;
  for (int s = 0; s < nsplit; ++s) {
    const float* rec = rec0 + s * part;
    const f32x4 tail = *reinterpret_cast<const f32x4*>(rec + D);  // m, den, count
    const float w = tail[0] == kNegInf ? 0.f : fast_exp2(tail[0] - m);
    den = den + w * tail[1];
    count += int(tail[2]);
    const f32x4 x = *reinterpret_cast<const f32x4*>(rec + 4 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = o[i] + w * x[i];
  }
  const int t = qb * kBlock + r % kBlock;
  if (p.counts && r % kBlock == 0 && c == 0) p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = count;
  if (t >= p.Tq) return;
  int64_t orow = int64_t(b) * p.Tq + t;
  if (p.out_index) {
    orow = p.out_index[orow];
    if (orow < 0 || orow >= p.out_rows) return;  // outside the output: not stored
  }
  u32x2 v;
  v[0] = pack_bf16x2(__fdiv_rn(o[0], den), __fdiv_rn(o[1], den));
  v[1] = pack_bf16x2(__fdiv_rn(o[2], den), __fdiv_rn(o[3], den));
  *reinterpret_cast<u32x2*>(p.out + (orow * p.H + h) * D + 4 * c) = v;
}

// Order of the R regular query tiles of a two-block launch whose routing
// masks are known before it (route_kernel): a tile's cost is its union of
// selected key blocks, and per (entry, head) the tiles are ranked by falling
// cost (ties by index) and dealt to the XCD slices of balanced_task in snake
// order (rank 0 .. 7 to XCDs 0 .. 7, ranks 8 .. 15 to XCDs 7 .. 0, ...; the R
// mod 8 cheapest to the XCDs with a leftover slot), each slice taking its
// tiles in falling cost.  Every XCD then holds about the same work of each
// head, the costly workgroups start first, and the grid's tail is short.
// order[bh NQB + slot] = the regular tile of that slot.  A permutation:
// results do not depend on it.
// kOrderParts workgroups per (entry, head): each forms every tile's cost
// (the mask words read eight at a time, so the loads overlap) and ranks one
// part of the tiles, kRankLanes adjacent lanes per tile, each counting over
// a strided share of the other tiles, their counts summed with shuffles.
constexpr int kOrderThreads = 1024;
constexpr int kOrderMaxTiles = 4096;
constexpr int kOrderParts = 8;
constexpr int kRankLanes = 8;
static_assert(kOrderThreads % kRankLanes == 0 && kWave % kRankLanes == 0, "rank groups stay inside a wave");

__global__ __launch_bounds__(kOrderThreads) void order_kernel(AttnParams p, int front, int F) {
  __shared__ uint32_t s_cost[kOrderMaxTiles];
  const int bh = blockIdx.x / kOrderParts, part = blockIdx.x % kOrderParts;
  const int ntiles = (p.NQB + 1) / 2, R = ntiles - front;
  const int stride = p.pair_stride ? min(p.pair_stride[bh], p.NQB) : 0;
  const uint32_t* mask = p.mask + int64_t(bh) * p.NQB * p.NW;
  for (int r = threadIdx.x; r < R; r += kOrderThreads) {
    const int t = front + r;
    const int a = slot_block(2 * t, p.NQB, stride), b = slot_block(2 * t + 1, p.NQB, stride);
    const uint32_t* ma = mask + int64_t(a) * p.NW;
    const uint32_t* mb = b < p.NQB ? mask + int64_t(b) * p.NW : ma;  // no partner: its own words
    uint32_t n = 0;
    int w = 0;
    for (; w + 8 <= p.NW; w += 8) {
      uint32_t m[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) m[u] = ma[w + u] | mb[w + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) n += __builtin_popcount(m[u]);
    }
    for (; w < p.NW; ++w) n += __builtin_popcount(ma[w] | mb[w]);
    s_cost[r] = n;
  }
  __syncthreads();
  const int base = R / kXcds, rem = R % kXcds;
  const int c = int((int64_t(F) + int64_t(bh) * rem) % kXcds);  // first XCD with a leftover slot
  const int chunk = (R + kOrderParts - 1) / kOrderParts;
  const int r0 = part * chunk, r1 = min(R, r0 + chunk);
  const int tasks = max(0, r1 - r0) * kRankLanes;  // whole rank groups: a group is all in or all out
  for (int task = threadIdx.x; task < tasks; task += kOrderThreads) {
    const int r = r0 + task / kRankLanes, sub = task % kRankLanes;
    const uint32_t cr = s_cost[r];
    int rank = 0;
    for (int q = sub; q < R; q += kRankLanes) {
      const uint32_t cq = s_cost[q];
      rank += (cq > cr || (cq == cr && q < r)) ? 1 : 0;
    }
#pragma unroll
    for (int off = 1; off < kRankLanes; off <<= 1) rank += __shfl_xor(rank, off);
    if (sub != 0) continue;
    int x, j;
    if (rank < kXcds * base) {
      const int round = rank / kXcds, q = rank % kXcds;
      x = (round & 1) ? kXcds - 1 - q : q;
      j = round;
    } else {
      x = (c + rank - kXcds * base) % kXcds;
      j = base;
    }
    const int extra_before = c + rem <= kXcds ? max(0, min(x, c + rem) - c)
                                              : max(0, x - c) + min(x, c + rem - kXcds);
    p.order[int64_t(bh) * p.NQB + x * base + extra_before + j] = r;
  }
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

template <int D, int G, bool SEG>
void launch_sol_variant(const AttnParams& p, hipStream_t stream) {
  // Grid of sol_task: the sink-holding tiles of every head (p.splits
  // workgroups each), then balanced_task's.
  const int ntiles = (p.NQB + G - 1) / G, front = std::min(p.q_sink_blocks, ntiles);
  const int split_tiles = sink_split_tiles(p.splits, p.q_sink_blocks, G, front);
  const unsigned grid = balanced_grid((split_tiles * (p.splits - 1) + front) * (p.B * p.H), p.B * p.H, ntiles - front);
  // Key blocks from pooled tile pairs (p.tiles) or straight from K / V rows.
  if (p.tiles) {
    if (p.k8)
      hipLaunchKernelGGL((sol_attention_kernel<D, G, kSolRing, true, true, SEG>), dim3(grid), dim3(128 * G), 0,
                         stream, p);
    else
      hipLaunchKernelGGL((sol_attention_kernel<D, G, kSolRing, false, true, SEG>), dim3(grid), dim3(128 * G), 0,
                         stream, p);
  } else {
    if (p.k8)
      hipLaunchKernelGGL((sol_attention_kernel<D, G, kSolRing, true, false, SEG>), dim3(grid), dim3(128 * G), 0,
                         stream, p);
    else
      hipLaunchKernelGGL((sol_attention_kernel<D, G, kSolRing, false, false, SEG>), dim3(grid), dim3(128 * G), 0,
                         stream, p);
  }
}

template <int D, int G>
void launch_sol_group(const AttnParams& p, hipStream_t stream) {
  // Key sequences beyond one routing segment take the segmented kernel.
  if (p.NKB > kMaxKeyBlocks)
    launch_sol_variant<D, G, true>(p, stream);
  else
    launch_sol_variant<D, G, false>(p, stream);
  const int front = std::min(p.q_sink_blocks, (p.NQB + G - 1) / G);
  const int split_tiles = sink_split_tiles(p.splits, p.q_sink_blocks, G, front);
  if (split_tiles > 0) {
    constexpr int kRows = kMergeThreads / (D / 4);
    const int64_t rows = int64_t(p.B) * p.H * split_tiles * G * kBlock;
    hipLaunchKernelGGL((sol_merge_kernel<D, G>), dim3(unsigned((rows + kRows - 1) / kRows)), dim3(kMergeThreads), 0,
                       stream, p, split_tiles);
  }
}

template <int D, int KS>
void launch_small(const AttnParams& p, hipStream_t stream) {
  const dim3 grid(unsigned(p.B * p.H * p.NQB)), block(128 * KS);
  if (p.tiles)
    hipLaunchKernelGGL((sol_small_kernel<D, KS, true, false>), grid, block, 0, stream, p);
  else if (!p.ctiles)
    hipLaunchKernelGGL((sol_small_kernel<D, KS, false, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sol_small_kernel<D, KS, false, false>), grid, block, 0, stream, p);
}

hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream) {
  // Routing first when its masks go to the routing workspace (beta = -inf
  // selects every block and needs none; without a workspace the attention
  // kernel routes tile by tile).
  if (p.force != 1 && p.mask) {
    const hipError_t err = launch_route(p, D, stream);
    if (err != hipSuccess) return err;
  }
  // Small launches: one query block per workgroup, key-split groups (the
  // caller passes no split workspace for them).  A forced workgroup form and
  // beta = -inf keep sol_attention_kernel, whose every-block-exact path
  // equals the dense kernel bit for bit.
  const int ks = p.workgroup_form == 0 && !p.k8 && p.splits == 1 && p.force != 1
                     ? small_key_split(int64_t(p.B) * p.H * p.NQB, p.NKB, D) : 0;
  if (ks) {
    if (D == 128)
      launch_small<128, 2>(p, stream);
    else
      launch_small<64, 4>(p, stream);
    return hipGetLastError();
  }
  int g = int64_t(p.B) * p.H * ((p.NQB + 1) / 2) < kSmallLaunchGroups ? 1 : 2;
  if (p.workgroup_form == 1 || p.workgroup_form == 2) g = p.workgroup_form;
  AttnParams q = p;
  q.order = nullptr;
  if (g == 2 && p.order && p.mask && p.force != 1 && p.splits == 1) {
    const int ntiles = (p.NQB + 1) / 2, front = std::min(p.q_sink_blocks, ntiles);
    if (ntiles - front > 0 && ntiles - front <= kOrderMaxTiles) {
      hipLaunchKernelGGL(order_kernel, dim3(unsigned(p.B * p.H * kOrderParts)), dim3(kOrderThreads), 0, stream, p,
                         front, front * p.B * p.H);
      const hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
      q.order = p.order;
    }
  }
  if (D == 128) {
    if (g == 1) launch_sol_group<128, 1>(q, stream); else launch_sol_group<128, 2>(q, stream);
  } else {
    if (g == 1) launch_sol_group<64, 1>(q, stream); else launch_sol_group<64, 2>(q, stream);
  }
  return hipGetLastError();
}

hipError_t launch_dense(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned grid = balanced_grid(0, p.B * p.H, (p.Tq + 127) / 128);
  if (D == 128) {
    if (p.tiles)
      hipLaunchKernelGGL((dense_attention_kernel<128, true>), dim3(grid), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dense_attention_kernel<128, false>), dim3(grid), dim3(256), 0, stream, p);
  } else {
    if (p.tiles)
      hipLaunchKernelGGL((dense_attention_kernel<64, true>), dim3(grid), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((dense_attention_kernel<64, false>), dim3(grid), dim3(256), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace sol
