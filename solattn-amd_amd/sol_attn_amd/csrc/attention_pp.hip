// Ping-pong SOL routed attention for gfx950: two query blocks per workgroup,
// eight waves, the blocks' common exact tiles streamed once for both and the
// rest in pairs, one wave of each block on every SIMD.
//
// Replaces the reference's `_threshold` (src/sol_attn_amd/kernels.py:52-64)
// and `_sol` (kernels.py:101-182) for launches large enough to fill the GPU;
// with every block exact it is also the dense control (`_dense`,
// kernels.py:67-98).
//
// Workgroup: 512 threads = 8 waves.  Wave w serves query-block slot
// g = w >> 2, key half kh = (w >> 1) & 1 (keys 32 kh .. +31 of every 64-key
// tile) and query half qh = w & 1 (queries 32 qh .. +31 of the block), with
// its own FP32 online-softmax state; the two key halves of a query are merged
// at the end.  The dispatcher deals a workgroup's waves to the four SIMDs
// round-robin, so waves w and w + 4 -- one of each slot -- share a SIMD.
// Slot 1 runs half a step behind slot 0: in every step a slot-0 wave computes
// S = K Q^T, the softmax and O += V P for the step's tile, while its SIMD
// partner first finishes the softmax and O += V P of its previous tile and
// then forms S of the current one.  Each wave's softmax (VALU) thus runs
// beside the other wave's matrix-core work.
//
// Tile stream, in steps (one workgroup barrier each):
//   1. centroid steps (finite or +inf beta): centroid tile c, 64 block
//      centroids, for both slots.  All eight waves first route the tile's
//      blocks for both query blocks -- proxy Qc . Kc_j against the Eq. 15
//      cutoff, strict >, then sink / local / plan protection
//      (kernels.py:118-143) -- into LDS bitmasks; after a barrier every wave
//      adds the unselected blocks' centroid terms, exp(s - m) * len_j with
//      value Vc_j (kernels.py:145-158), through the same tile pipeline;
//   2. shared steps: the blocks both query blocks selected, ascending, one
//      tile for both slots;
//   3. pair steps: each slot's remaining selected blocks, ascending, one tile
//      per slot per step (a slot whose list is done waits).
// The tiles land in a four-slot LDS pool by global_load_lds DMA issued up to
// four tiles ahead; a tile's slot is refilled once the step after its last
// use has passed its barrier.  The step order is a fixed function of the
// routing masks, so results are deterministic.
#include <algorithm>
#include <type_traits>

#include "attn_common.h"

namespace sol {

namespace {

constexpr int kPPThreads = 512;
constexpr int kPool = 4;             // LDS tile slots
constexpr int kCentTag = 1 << 20;    // tile reference of centroid tile c: kCentTag | c
constexpr int kNoTile = -1;

constexpr int kMaskWords = kMaxKeyBlocks / 32;

// Routing bitmasks of the workgroup's two query-block slots (bit j: block j
// exact).  At namespace scope, so that the step cursors address them by
// constant LDS offsets instead of carrying pointers.
__shared__ uint32_t pp_mask[2][kMaskWords];

struct StepPair {
  int a, b;  // tile references of slots 0 and 1 (kNoTile: the slot waits)
};

// Ascending bits of one of three sets over the two slots' routing masks:
// kind 0 both, 1 slot 0 only, 2 slot 1 only.  Wave-uniform.
template <int KIND>
struct BitCursor {
  int word, last;
  uint32_t bits;

  __device__ __forceinline__ static uint32_t load(int w) {
    const uint32_t x = pp_mask[0][w], y = pp_mask[1][w];
    const uint32_t v = KIND == 0 ? (x & y) : (KIND == 1 ? (x & ~y) : (y & ~x));
    return uint32_t(__builtin_amdgcn_readfirstlane(v));
  }
  __device__ __forceinline__ void init(int nwords) {
    word = 0;
    last = nwords - 1;
    bits = load(0);
  }
  __device__ __forceinline__ int next() {
    while (bits == 0 && word < last) bits = load(++word);
    if (bits == 0) return kNoTile;
    const int j = word * 32 + __builtin_ctz(bits);
    bits &= bits - 1u;
    return j;
  }
};

// The step sequence of a workgroup.  The consumer and the DMA issuer each run
// one copy; the issuer runs ahead and may not enter the exact steps before
// the routing masks are complete.
struct StepGen {
  int nwords, nct, c, phase;  // phase 0 centroid, 1 shared, 2 pairs
  bool two;                   // slot 1 holds a query block
  BitCursor<0> shared;
  BitCursor<1> only0;
  BitCursor<2> only1;

  __device__ __forceinline__ void init(int nw, int centroid_tiles, bool slot1) {
    nwords = nw;
    nct = centroid_tiles;
    c = 0;
    two = slot1;
    phase = 0;
  }
  __device__ __forceinline__ bool needs_masks() const { return phase == 0 && c >= nct; }
  __device__ __forceinline__ StepPair next() {
    if (phase == 0) {
      if (c < nct) {
        const int r = kCentTag | c++;
        return {r, two ? r : kNoTile};
      }
      phase = 1;
      shared.init(nwords);
      only0.init(nwords);
      only1.init(nwords);
    }
    if (phase == 1) {
      const int j = shared.next();
      if (j != kNoTile) return {j, j};
      phase = 2;
    }
    const int a = only0.next();
    const int b = only1.next();
    return {a, b};
  }
};

__device__ __forceinline__ bool is_centroid(int ref) { return ref >= kCentTag; }

// Waits until at most `ahead` tiles' DMA (the newest ones) are still in flight.
template <int kRounds>
__device__ __forceinline__ void wait_tiles(int ahead) {
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

// Initial scores of this wave's 32-key half of tile `ref`: 0 for present
// keys, -inf for keys past the sequence (exact tail block) or for blocks the
// query block selected (centroid tiles), log2(len_j) / c for the centroids it
// approximates, so that exp2(s c - m) carries len_j (kernels.py:153-155).
__device__ __forceinline__ f32x16 half_bias(int ref, const uint32_t* mask, int kh, int hh, int tk, int nkb,
                                            float c) {
  f32x16 bias;
  if (is_centroid(ref)) {
    const int ct = ref - kCentTag;
    const uint64_t lane_approx = tile_approx(mask, ct, nkb) >> (32 * kh + 4 * hh);
    const float inv_c = 1.f / c;
    const int lane_tokens = tk - kBlock * (kBlock * ct + 32 * kh + 4 * hh);  // from the lane's first block
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = tile_row(0, e, 0);
      const int len = min(kBlock, lane_tokens - kBlock * row);
      bias[e] = ((lane_approx >> row) & 1u) ? __builtin_amdgcn_logf(float(max(len, 1))) * inv_c : kNegInf;
    }
  } else {
    const int lane_keys = tk - ref * kBlock - 32 * kh - 4 * hh;  // keys from the lane's first row on
#pragma unroll
    for (int e = 0; e < 16; ++e) bias[e] = tile_row(0, e, 0) < lane_keys ? 0.f : kNegInf;
  }
  return bias;
}

// K fragments of the wave's 32-key half of the tile in `buf`.
template <int D>
__device__ __forceinline__ void half_keys(const uint16_t* buf, int kh, const FragLane<D>& fl,
                                          u32x4 (&kf)[Shape<D>::KT]) {
#pragma unroll
  for (int ks = 0; ks < Shape<D>::KT; ++ks) kf[ks] = fl.k(buf, kh, ks);
}

// S^T of a 32-key half (32 keys x 32 queries) from its K fragments,
// accumulated onto `s`.
template <int D>
__device__ __forceinline__ f32x16 half_scores(const u32x4 (&kf)[Shape<D>::KT], const bf16x8 (&qf)[Shape<D>::KT],
                                              f32x16 s) {
#pragma unroll
  for (int ks = 0; ks < Shape<D>::KT; ++ks) s = mfma32x32x16(as_bf16x8(kf[ks]), qf[ks], s);
  return s;
}

template <int D>
__device__ __forceinline__ void half_values(const uint16_t* buf, int kh, const FragLane<D>& fl,
                                            u32x4 (&vf)[2][Shape<D>::DT]) {
#pragma unroll
  for (int c4 = 0; c4 < 2; ++c4)
#pragma unroll
    for (int dt = 0; dt < Shape<D>::DT; ++dt) vf[c4][dt] = fl.v(buf, kh, c4, dt);
}

// Online softmax of a half's scores, then O^T += V^T P^T (kernels.py:159-178).
template <int D>
__device__ __forceinline__ void half_update(State<D>& st, const f32x16& s, const u32x4 (&vf)[2][Shape<D>::DT],
                                            float c) {
  HalfSoftmax<D> h;
  h.s = s;
#pragma unroll
  for (int k = 0; k < 8; ++k) h.stage(k, st, c);
  if (h.rescale) rescale_acc<D>(st, h.alpha);
#pragma unroll
  for (int c4 = 0; c4 < 2; ++c4)
#pragma unroll
    for (int dt = 0; dt < Shape<D>::DT; ++dt)
      st.acc[dt] = mfma32x32x16(as_bf16x8(vf[c4][dt]), h.pb(c4), st.acc[dt]);
}

// Pulls the 16-bit piece at bits 0, 4, .., 60 of a ballot (one bit per lane
// quad) down to bits 0 .. 15.
__device__ __forceinline__ uint32_t quad_bits(uint64_t x) {
  x &= 0x1111111111111111ull;
  x = (x | (x >> 3)) & 0x0303030303030303ull;
  x = (x | (x >> 6)) & 0x000F000F000F000Full;
  x = (x | (x >> 12)) & 0x000000FF000000FFull;
  x = (x | (x >> 24)) & 0xFFFFull;
  return uint32_t(x);
}

}  // namespace

// __launch_bounds__(512, 2): two waves per SIMD, one workgroup per CU, 256
// registers per wave.
template <int D, bool DENSE>
__global__ __launch_bounds__(kPPThreads, 2) void sol_pp_kernel(AttnParams p) {
  using S = Shape<D>;
  using TL = TileLayout<D>;
  constexpr int NT = kPPThreads;
  constexpr int kRounds = S::TILE / 8 / NT;  // DMA rounds per tile per wave
  static_assert(kPool * S::TILE >= 2 * kBlock * S::KS, "Q staging fits in the pool");
  static_assert(kPool * S::TILE * 2 >= 4 * (S::DT * 16 + 2) * kWave * 4, "key-half merge fits in the pool");
  __shared__ __align__(16) uint16_t pool[kPool * S::TILE];  // Q staging, tile pool, key-half merge
  __shared__ float s_qm[2][D];
  __shared__ float s_red[2][4];
  __shared__ float s_cut[2];

  const int ntiles = (p.NQB + 1) / 2;
  const TileTask task = DENSE ? xcd_task(blockIdx.x, ntiles)
                              : sol_task(blockIdx.x, ntiles, min(p.q_sink_blocks, ntiles), p.B * p.H);
  if (task.bh < 0) return;
  const int bh = task.bh;
  const int h = bh % p.H, b = bh / p.H;
  const int64_t head = int64_t(b) * p.H + h;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, hh = lane >> 5;
  const int g = wave >> 2, kh = (wave >> 1) & 1, qh = wave & 1;
  const int stride = (!DENSE && p.pair_stride) ? min(p.pair_stride[bh], p.NQB) : 0;
  const int qb0 = slot_block(2 * task.tile, p.NQB, stride);
  const int qb1 = slot_block(2 * task.tile + 1, p.NQB, stride);
  auto qb_of = [&](int s) { return s ? qb1 : qb0; };
  const bool two = qb1 < p.NQB;  // slot 0 always holds a query block
  const int qb = qb_of(g);
  const bool live = qb < p.NQB;
  const int tk = batch_tokens(p.klen, b, p.Tk);
  const int nkb = (tk + kBlock - 1) / kBlock;
  const int nct = (nkb + kBlock - 1) / kBlock;
  const int nwords = (nkb + 31) / 32;
  const float scale_log2 = p.scale_log2;
  const int force = DENSE ? 1 : p.force;

  // 1. Q tiles of both slots -> LDS -> register fragments.
  for (int idx = tid; idx < 2 * kBlock * S::DC; idx += NT) {
    const int r = idx / S::DC, c = idx % S::DC;
    const int t = qb_of(r >= kBlock) * kBlock + r % kBlock;  // >= Tq for an empty slot
    const u32x4 x = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(pool + r * S::KS + 8 * c) = x;
  }
  __syncthreads();
  bf16x8 qf[S::KT];
  const int myq = 32 * qh + col;  // query inside the block
  {
    const uint16_t* qrow = pool + (g * kBlock + myq) * S::KS;
#pragma unroll
    for (int ks = 0; ks < S::KT; ++ks)
      qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(qrow + ks * 16 + 8 * hh));
  }

  // 2. Query means (torch's cascade order) and cutoffs of both slots.
  if (force == 0) {
    const int gs = tid / D, f = tid % D;  // slot, feature (threads below 2 D)
    if (tid < 2 * D) {
      const int q0 = qb_of(gs);
      const int qlen = q0 < p.NQB ? min(kBlock, p.Tq - q0 * kBlock) : 1;
      float tot = 0.f;
      for (int c = 0; c < 4; ++c) {
        float sum = 0.f;
        for (int i = 0; i < 16; ++i) {
          const int r = 16 * c + i;
          if (r < qlen) sum = __fadd_rn(sum, bf16_bits_to_f32(pool[(gs * kBlock + r) * S::KS + f]));
        }
        tot = __fadd_rn(tot, sum);
      }
      s_qm[gs][f] = __fdiv_rn(tot, float(qlen));
    }
    if (tid < 8) s_red[tid >> 2][tid & 3] = 0.f;
    __syncthreads();
    float a = 0.f, q2 = 0.f;
    if (tid < 2 * D) {
      const float qm = s_qm[gs][f];
      a = qm * p.mean[head * D + f];
      if (p.cov) {
        // Full covariance: this feature's term of Qc^T cov Qc.
        const float* row = p.cov + (head * D + f) * D;
        float sq = 0.f;
        for (int e = 0; e < D; ++e) sq = fmaf(row[e], s_qm[gs][e], sq);
        q2 = qm * sq;
      } else {
        q2 = qm * qm * p.var[head * D + f];
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      a += __shfl_xor(a, off);
      q2 += __shfl_xor(q2, off);
    }
    if (lane == 0 && tid < 2 * D) {
      const int part = (tid % D) / kWave;  // which 64-feature part of the slot
      s_red[gs][part] = a;
      s_red[gs][2 + part] = q2;
    }
    __syncthreads();
    if (tid < 2) {
      const float quad = s_red[tid][2] + s_red[tid][3];  // the full quadratic form may round below 0
      s_cut[tid] = (s_red[tid][0] + s_red[tid][1]) + p.beta * sqrtf(p.cov ? fmaxf(quad, 0.f) : quad);
    }
  }
  if (force == 1) {
    // Every valid block exact (beta = -inf, or the dense control).
    for (int i = tid; i < 2 * nwords; i += NT) {
      const int gs = i / nwords, w = i % nwords;
      const int nvalid = min(32, nkb - 32 * w);
      pp_mask[gs][w] = qb_of(gs) < p.NQB ? (nvalid == 32 ? ~0u : ((1u << nvalid) - 1u)) : 0u;
    }
    if (!DENSE && p.dbg_selected)
      for (int i = tid; i < 2 * nkb; i += NT) {
        const int gs = i / nkb, j = i % nkb;
        if (qb_of(gs) < p.NQB) p.dbg_selected[((int64_t(b) * p.NQB + qb_of(gs)) * p.H + h) * p.NKB + j] = 1;
      }
  }
  __syncthreads();  // cutoffs and masks published; the Q staging is dead
  if (!DENSE && p.dbg_cutoff && tid < 2 && qb_of(tid) < p.NQB)
    p.dbg_cutoff[(int64_t(b) * p.NQB + qb_of(tid)) * p.H + h] =
        force == 0 ? s_cut[tid] * p.scale : (force == 1 ? kNegInf : -kNegInf);

  State<D> st;
  state_init(st);
  const uint32_t pool_lds = lds_address(pool);
  const uint16_t* tiles = p.tiles + head * p.NKB * S::TILE;
  const uint16_t* ctiles = DENSE ? nullptr : p.ctiles + head * p.NCT * S::TILE;
  auto source = [&](int ref) {
    return is_centroid(ref) ? ctiles + int64_t(ref - kCentTag) * S::TILE : tiles + int64_t(ref) * S::TILE;
  };
  const int centroid_tiles = force == 1 ? 0 : nct;

  // DMA issuer: the stream's tiles in order, into slot (index % kPool).
  StepGen ig;
  ig.init(nwords, centroid_tiles, two);
  int issued = 0, pending = kNoTile;
  bool issue_done = false;
  bool routed = centroid_tiles == 0;
  auto issue_upto = [&](int limit) {
    while (issued < limit) {
      int ref = pending;
      if (ref != kNoTile) {
        pending = kNoTile;
      } else {
        if (issue_done || (ig.needs_masks() && !routed)) break;
        const StepPair sp = ig.next();
        if (sp.a == kNoTile && sp.b == kNoTile) {
          issue_done = true;
          break;
        }
        ref = sp.a != kNoTile ? sp.a : sp.b;
        if (sp.a != kNoTile && sp.b != kNoTile && sp.b != sp.a) pending = sp.b;
      }
      TileRefill<D, NT>(source(ref), pool_lds + uint32_t((issued % kPool) * S::TILE * 2), wave, lane).all();
      ++issued;
    }
  };
  issue_upto(kPool);

  const uint32_t* my_mask = pp_mask[g];
  const int64_t dbg_base = (int64_t(b) * p.NQB) * p.H;
  // The step loop, instantiated once per slot role so that each keeps only
  // its own registers live: slot 0 computes a step's tile within the step;
  // slot 1 carries its previous tile's scores and V^T fragments into the
  // next step.
  auto stream = [&](auto role) {
    constexpr bool kLag = decltype(role)::value;
    StepGen cg;
    cg.init(nwords, centroid_tiles, two);
    int consumed = 0;
    f32x16 s_prev = zero16();
    u32x4 v_prev[2][S::DT];
    bool has_prev = false;
    for (;;) {
      const StepPair sp = cg.next();
      if (sp.a == kNoTile && sp.b == kNoTile) break;
      const int na = sp.a != kNoTile ? 1 : 0;
      const int nb = (sp.b != kNoTile && sp.b != sp.a) ? 1 : 0;
      const int slot_a = consumed % kPool;
      const int slot_b = sp.b == sp.a ? slot_a : (consumed + na) % kPool;
      wait_tiles<kRounds>(issued - consumed - na - nb);
      ring_barrier();  // this step's tiles are in LDS; the previous step's slots are free
      issue_upto(consumed + kPool);
      const bool cent = !DENSE && is_centroid(sp.a);
      if (cent) {
        // Routing of centroid tile ct for both slots: thread = (slot, block
        // row, feature quarter); proxies summed over the quarter's lane quad.
        const int ct = sp.a - kCentTag;
        const uint16_t* buf = pool + slot_a * S::TILE;
        const int pair = tid >> 2, quarter = tid & 3;
        const int gs = pair >> 6, r = pair & 63;
        const int j = kBlock * ct + r;
        const int qs = qb_of(gs);
        bool sel = false;
        float proxy = 0.f;
        if (force == 0) {
          constexpr int QC = S::DC / 4;  // 16-byte chunks per quarter
          float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int cc = 0; cc < QC; ++cc) {
            const int chunk = quarter * QC + cc;
            const u32x4 x = *reinterpret_cast<const u32x4*>(buf + TL::k_offset(r, chunk));
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t w = x[e >> 1];
              part[e & 3] = fmaf(s_qm[gs][8 * chunk + e],
                                 bf16_bits_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu)), part[e & 3]);
            }
          }
          proxy = (part[0] + part[1]) + (part[2] + part[3]);
          proxy += __shfl_xor(proxy, 1);
          proxy += __shfl_xor(proxy, 2);
        }
        if (qs < p.NQB && j < nkb) {
          if (force == 0) sel = proxy > s_cut[gs];
          sel = sel || (p.local_blocks >= 0 && abs(j - qs) <= p.local_blocks) || j < p.kv_sink_blocks ||
                qs < p.q_sink_blocks;
          if (p.protection) sel = sel || p.protection[(int64_t(b) * p.NQB + qs) * p.NKB + j] != 0;
          if (quarter == 0) {
            const int64_t row = (dbg_base + int64_t(qs) * p.H + h) * p.NKB + j;
            if (p.dbg_proxy && force == 0) p.dbg_proxy[row] = proxy * p.scale;
            if (p.dbg_selected) p.dbg_selected[row] = sel ? 1 : 0;
          }
        }
        const uint32_t bits = quad_bits(__ballot(sel));
        if (lane == 0) reinterpret_cast<uint16_t*>(pp_mask[wave >> 2])[4 * ct + (wave & 3)] = uint16_t(bits);
        lds_barrier();  // publishes the tile's mask words
        if (ct == nct - 1) {
          routed = true;
          issue_upto(consumed + kPool);  // the exact tiles can be fetched now
        }
      }
      const FragLane<D> fl(fresh(col), fresh(hh));
      // Every LDS fragment read of a step is issued before the matrix-core
      // work that consumes it (chunk_end keeps the order), so one read
      // latency is paid per step instead of one per MFMA.
      if constexpr (!kLag) {
        if (sp.a != kNoTile) {
          const uint16_t* buf = pool + slot_a * S::TILE;
          u32x4 kf[S::KT], vf[2][S::DT];
          half_keys<D>(buf, kh, fl, kf);
          half_values<D>(buf, kh, fl, vf);
          const f32x16 init = cent || (sp.a + 1) * kBlock > tk
                                  ? half_bias(sp.a, my_mask, kh, hh, tk, nkb, scale_log2) : zero16();
          chunk_end();
          const f32x16 s = half_scores<D>(kf, qf, init);
          half_update<D>(st, s, vf, scale_log2);
        }
      } else {
        const bool next = sp.b != kNoTile;
        const uint16_t* buf = pool + slot_b * S::TILE;
        u32x4 kf[S::KT];
        if (next) half_keys<D>(buf, kh, fl, kf);
        chunk_end();
        if (has_prev) half_update<D>(st, s_prev, v_prev, scale_log2);
        has_prev = next;
        if (next) {
          const f32x16 init = (!DENSE && is_centroid(sp.b)) || (sp.b + 1) * kBlock > tk
                                  ? half_bias(sp.b, my_mask, kh, hh, tk, nkb, scale_log2) : zero16();
          s_prev = half_scores<D>(kf, qf, init);
          half_values<D>(buf, kh, fl, v_prev);
        }
      }
      consumed += na + nb;
    }
    wait_vmcnt<0>();
    if (kLag && has_prev) half_update<D>(st, s_prev, v_prev, scale_log2);
  };
  if (g == 0)
    stream(std::false_type{});
  else
    stream(std::true_type{});
  if (!DENSE && p.counts && tid < 2 && qb_of(tid) < p.NQB) {
    int nsel = 0;
    for (int w = 0; w < nwords; ++w) nsel += __builtin_popcount(pp_mask[tid][w]);
    p.counts[(int64_t(b) * p.NQB + qb_of(tid)) * p.H + h] = nsel;
  }

  // 4. Merge the two key halves of every query (through LDS) and store.
  __syncthreads();  // every wave is done with the pool
  constexpr int kMerge = S::DT * 16 + 2;  // floats per lane: acc, m, den
  float* mbuf = reinterpret_cast<float*>(pool) + (g * 2 + qh) * kMerge * kWave + lane;
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) mbuf[(dt * 16 + e) * kWave] = st.acc[dt][e];
    mbuf[(S::DT * 16) * kWave] = st.m;
    mbuf[(S::DT * 16 + 1) * kWave] = st.den;
  }
  __syncthreads();
  if (kh == 0 && live) {
    const float m1 = mbuf[(S::DT * 16) * kWave];
    const float d1 = mbuf[(S::DT * 16 + 1) * kWave];
    const float m = fmaxf(st.m, m1);
    const float ref = m == kNegInf ? 0.f : m;
    const float a0 = st.m == kNegInf ? 0.f : fast_exp2(st.m - ref);
    const float a1 = m1 == kNegInf ? 0.f : fast_exp2(m1 - ref);
#pragma unroll
    for (int dt = 0; dt < S::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) st.acc[dt][e] = st.acc[dt][e] * a0 + mbuf[(dt * 16 + e) * kWave] * a1;
    st.den = st.den * a0 + d1 * a1;
    store_output<D>(p, b, h, qb * kBlock + myq, hh, st);
  }
}

hipError_t launch_sol_pp(const AttnParams& p, int D, hipStream_t stream) {
  const int ntiles = (p.NQB + 1) / 2, front = std::min(p.q_sink_blocks, ntiles);
  const unsigned grid = unsigned(front) * unsigned(p.B * p.H) + xcd_grid(p.B * p.H, ntiles - front);
  if (D == 128)
    hipLaunchKernelGGL((sol_pp_kernel<128, false>), dim3(grid), dim3(kPPThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((sol_pp_kernel<64, false>), dim3(grid), dim3(kPPThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_dense_pp(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned grid = xcd_grid(p.B * p.H, (p.NQB + 1) / 2);
  if (D == 128)
    hipLaunchKernelGGL((sol_pp_kernel<128, true>), dim3(grid), dim3(kPPThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((sol_pp_kernel<64, true>), dim3(grid), dim3(kPPThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
