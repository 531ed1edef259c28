// Device building blocks of the SOL attention kernels (attention.hip): the workgroup -> query-tile maps, the FP32 online-softmax
// state of a wave, the LDS DMA tile refill, the MFMA operand reads from the
// swizzled tiles, and the output store.
#pragma once

#include "sol_device.h"
#include "sol_internal.h"

#define SOL_LDS __attribute__((address_space(3)))

namespace sol {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

constexpr int kXcds = 8;

// Workgroup ids are dealt round-robin over the 8 XCDs.  The id -> (head, query
// tile) map keeps every XCD on the SAME head at the same time, each on its own
// contiguous slice of that head's query tiles: neighbouring tiles share that
// XCD's L2, and the tiles of one head (43 MB at 84,672 tokens) are the whole
// live set of the memory-side cache.  The first F ids (a SOL launch's
// query-sink tiles, sol_task) go ahead of that map; after them, XCD x's
// workgroups take, head after head, its slice of the head's R tiles: floor(R
// / 8) tiles, one more for the XCDs that the R mod 8 leftover tiles of each
// head are dealt to -- round-robin, continuing from the F front ids -- so that
// every XCD holds the same number of workgroups to within one.  (Equal
// ceil(R / 8) slices with the last XCD short left 7 XCDs a workgroup round
// more than the eighth when R mod 8 != 0, or when the front ids fell on
// them: at 32,768 tokens x 4 heads with 128-token sinks, 129 workgroups
// against 64 slots per XCD.)  Ids past an XCD's count return -1 (idle).
struct TileTask {
  int bh, tile;
  int split = 0;  // key-range part of a split front tile (sol_task)
};

// Regular workgroup id i >= F: (head, tile in [0, R)) as described above.
__device__ __forceinline__ TileTask balanced_task(int i, int F, int heads, int R) {
  const int x = i % kXcds, k = i / kXcds;
  const int fx = F > x ? (F - x + kXcds - 1) / kXcds : 0;  // front ids of XCD x
  const int kr = k - fx;                                    // its regular index
  const int base = R / kXcds, rem = R % kXcds;
  const int r0 = ((x - F) % kXcds + kXcds) % kXcds;  // leftover e goes to XCD (F + e) % 8
  // XCD x's regular workgroups in heads [0, h).
  auto cum = [&](int h) {
    const int n = h * rem;
    return h * base + (n > r0 ? (n - 1 - r0) / kXcds + 1 : 0);
  };
  int h = R > 0 ? min(heads, int(int64_t(kr) * kXcds / R)) : heads;
  while (h > 0 && cum(h) > kr) --h;
  while (h < heads && cum(h + 1) <= kr) ++h;
  if (h >= heads || kr < 0) return TileTask{-1, 0};
  // Start of XCD x's slice of head h: the slices of XCDs 0 .. x-1, of which
  // those in [c, c + rem) (mod 8) hold one leftover tile more.
  const int c = (F + h * rem) % kXcds;
  const int extra_before = c + rem <= kXcds ? max(0, min(x, c + rem) - c)
                                            : max(0, x - c) + min(x, c + rem - kXcds);
  return TileTask{h, x * base + extra_before + (kr - cum(h))};
}

// Workgroups of a launch of F front ids and `heads` x R regular tiles: every
// XCD's count, rounded up, eight times.
__host__ __device__ inline unsigned balanced_grid(int F, int heads, int R) {
  const int64_t total = int64_t(F) + int64_t(heads) * R;
  return unsigned(kXcds * ((total + kXcds - 1) / kXcds));
}

// SOL launches dispatch the first `front` query tiles of every (entry, head)
// ahead of the rest, head-interleaved.  With query sinks those tiles hold the
// sink query blocks, whose workgroups stream every key block and run several
// times longer than the others; behind the regular map the last heads' ones
// would start late and set the kernel's end (2 x 4,096 tokens x 16 heads with
// 128-token sinks: 251 -> 163 us).  The first `split_tiles` of them (<=
// front) are `splits` workgroups each, one per key range (split_range), whose
// partial states sol_merge_kernel combines.  The remaining tiles follow
// balanced_task.
__device__ __forceinline__ TileTask sol_task(int i, int ntiles, int front, int split_tiles, int heads,
                                             int splits) {
  const int nsplit = split_tiles * heads * splits;
  if (i < nsplit) {
    const int j = i / heads;
    return TileTask{i % heads, j / splits, j % splits};
  }
  const int nrest = (front - split_tiles) * heads;
  if (i - nsplit < nrest) return TileTask{(i - nsplit) % heads, split_tiles + (i - nsplit) / heads};
  TileTask t = balanced_task(i, nsplit + nrest, heads, ntiles - front);
  t.tile += front;
  return t;
}

// Query-sink tiles split by key range (sol_task) when a launch is split: the
// tiles of sink blocks [0, 2 floor(q_sink_blocks / 2)).  With adjacent
// pairing those tiles hold sink blocks only, in either workgroup form, so
// whether a query block is split depends on its index alone and both forms
// stay bit-identical.  A split launch pairs adjacent blocks (it ignores
// pair_stride).
__host__ __device__ inline int sink_split_tiles(int splits, int q_sink_blocks, int G, int front) {
  return splits > 1 ? min(front, (q_sink_blocks / 2 * 2) / G) : 0;
}

// Key blocks [lo, hi) of part s of n of a key sequence of nkb blocks.
__device__ __forceinline__ int2 split_range(int s, int n, int nkb) {
  return int2{int(int64_t(s) * nkb / n), int(int64_t(s + 1) * nkb / n)};
}



template <int D>
struct Shape {
  static constexpr int KS = D + 8;   // Q staging row stride (elements)
  static constexpr int DC = D / 8;   // 16-byte chunks per row
  static constexpr int KT = D / 16;  // MFMA k-steps over the head dimension
  static constexpr int DT = D / 32;  // 32-row output tiles over the head dimension
  static constexpr int TILE = 2 * kBlock * D;  // K + V tile elements per 64-key tile
};

// One wave's FP32 online-softmax state for its 32 queries (one per lane pair).
template <int D>
struct State {
  f32x16 acc[Shape<D>::DT];  // O^T: rows = features, column = this lane's query
  float m;                   // running max, log2 units (-inf: nothing yet)
  float den;                 // partial denominator over this lane's key rows
};

// Floats per query row of a split workgroup's partial state: acc (D), m,
// den, count, padding (sol_attention_kernel, sol_merge_kernel).
template <int D>
constexpr int kPartialRow = D + 4;

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
// barrier.  M0 (the LDS base register of the DMA) is declared clobbered
// rather than saved and restored around every DMA (two scalar instructions
// per DMA fewer; a refill is 8 DMAs per tile).  M0 is a reserved register,
// so hipcc warns that the clobber is not honoured: the compiler keeps no
// value of its own live in M0 across these statements.  In the kernels built
// from this file no instruction other than these DMAs reads M0 (checked in
// the device assembly, `--cuda-device-only -S`), so nothing relies on it.
__device__ __forceinline__ void dma16(uint64_t sbase, uint32_t lane_bytes, uint32_t m) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(m), "v"(lane_bytes), "s"(sbase)
      : "memory", "m0");
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

// Key blocks DMA'd into an LDS slot as a K + V tile pair (TileLayout)
// straight from the caller's K and V rows ("rows mode"; the other source is
// a pooled tile pair array, TileRefill).  Each round moves RPR = NT 16 / (2 D)
// key rows of K (or V): wave w's 1 KB piece of the slot, lane l's 16 bytes at
// LDS byte 16 (r NT + 64 w + l), is the chunk that position holds in the
// tile layout, so lane l reads row r RPR + (its round-0 row), chunk (its
// chunk).  The per-lane byte offsets klane / vlane (row * row stride +
// 16 chunk) are the same in every round, except for the K swizzle of
// D = 128 with 128 threads, whose rounds alternate klane / klane_odd.  The
// sequence's partial last block is read shifted back to rows Tk - 64 ..
// Tk - 1 (all present; Tk >= 64 in rows mode), so its keys sit in the
// tile's last Tk - 64 (NKB - 1) rows and the rows before them, keys of the
// previous block, are masked out by the consumer.
template <int D, int NT>
struct KvRows {
  static constexpr int kHalfRounds = kBlock * D * 2 / 16 / NT;  // DMA rounds per K (or V) tile
  static constexpr int kRowsPerRound = NT * 16 / (2 * D);
  static constexpr bool kOddK = D == 128 && NT == 128;          // K swizzle period of two rounds
  uint64_t k, v;            // byte address of key row 0 of this (entry, head)
  uint32_t stk, stv;        // bytes between key rows (token strides below 2^24 elements)
  int last, last_row;       // the partial last block (-1: none) and its first row
  uint32_t klane, vlane, klane_odd;  // klane_odd: kOddK only
};

template <int D, int NT>
__device__ __forceinline__ KvRows<D, NT> kv_rows(const AttnParams& p, int b, int h, int tid) {
  using TL = TileLayout<D>;
  using Src = KvRows<D, NT>;
  Src s;
  s.stk = uint32_t(p.k.st * 2);
  s.stv = uint32_t(p.v.st * 2);
  s.k = uniform64(reinterpret_cast<uint64_t>(p.k.base + int64_t(b) * p.k.sb + int64_t(h) * p.k.sh));
  s.v = uniform64(reinterpret_cast<uint64_t>(p.v.base + int64_t(b) * p.v.sb + int64_t(h) * p.v.sh));
  s.last = p.Tk % kBlock ? p.Tk / kBlock : -1;
  s.last_row = p.Tk - kBlock;
  const int w = tid >> 6, l = tid & 63;
  // K, row-major: the wave's 1 KB piece holds 512 / D rows.
  const int krow = w * (512 / D) + l / (D / 8), kpc = l % (D / 8);
  s.klane = uint32_t(krow * int64_t(s.stk) + 16 * (kpc ^ TL::k_swizzle(krow)));
  s.klane_odd = Src::kOddK ? uint32_t(krow * int64_t(s.stk) + 16 * (kpc ^ TL::k_swizzle(krow + Src::kRowsPerRound)))
                           : s.klane;
  // V, row quads of 8 D bytes: position 16 m of quad q holds row
  // 4 q + ((m >> 2) & 3), chunk 4 (m >> 4) + (m & 3).
  const int pos = w * 1024 + 16 * l;
  const int q = pos / (8 * D), m = (pos % (8 * D)) / 16;
  s.vlane = uint32_t((4 * q + ((m >> 2) & 3)) * int64_t(s.stv) + 16 * (4 * (m >> 4) + (m & 3)));
  return s;
}

// DMA of key block j from rows into the LDS slot at dst_lds (wave w's piece
// of round r at dst_lds + 1024 w + 16 r NT): the K rounds, then the V
// rounds; issued whole or a few rounds at a time, as TileRefill.
template <int D, int NT>
struct RowRefill {
  using Src = KvRows<D, NT>;
  static constexpr int kHalf = Src::kHalfRounds;
  static constexpr int kRounds = 2 * kHalf;
  uint64_t ksrc, vsrc;
  uint32_t kstep, vstep;
  uint32_t klane, vlane, klane_odd;
  uint32_t lds;

  __device__ __forceinline__ RowRefill(const Src& src, int j, uint32_t dst_lds, int wave)
      : klane(src.klane), vlane(src.vlane), klane_odd(src.klane_odd) {
    const uint32_t row = uint32_t(j == src.last ? src.last_row : j * kBlock);  // < 2^30
    ksrc = uniform64(src.k + uint64_t(row) * src.stk);   // 32 x 32 -> 64-bit product
    vsrc = uniform64(src.v + uint64_t(row) * src.stv);
    kstep = Src::kRowsPerRound * src.stk;
    vstep = Src::kRowsPerRound * src.stv;
    lds = uint32_t(__builtin_amdgcn_readfirstlane(dst_lds + uint32_t(wave) * (kWave * 16)));
  }
  __device__ __forceinline__ void round(int r) const {
    if (r < kHalf) {
      const uint32_t lane = (Src::kOddK && (r & 1)) ? klane_odd : klane;
      dma16(ksrc + uint64_t(uint32_t(r) * kstep), lane, lds + uint32_t(r * NT * 16));
    } else {
      const int rv = r - kHalf;
      dma16(vsrc + uint64_t(uint32_t(rv) * vstep), vlane, lds + uint32_t(TileLayout<D>::kElems * 2 + rv * NT * 16));
    }
  }
  __device__ __forceinline__ void all() const {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) round(r);
  }
  template <int N>
  __device__ __forceinline__ void after_step(int k) const {
#pragma unroll
    for (int r = k * kRounds / N; r < (k + 1) * kRounds / N; ++r) round(r);
  }
};

// DMA for the quantised-QK experiment's exact tiles: the INT8 K tile of a
// key block (64 rows x D bytes, contiguous in the INT8 tile array) at the
// slot's start, then the block's V tile as the BF16 refill V moves it (Kv: a
// RowRefill, or a TileRefill of the block's tile pair).  Rounds: the K8
// rounds, then the V rounds.
template <int D, int NT, typename Kv>
struct Q8Refill {
  static constexpr int kK8Rounds = kBlock * D / 16 / NT;
  static constexpr int kVRounds = Kv::kRounds / 2;
  static constexpr int kRounds = kK8Rounds + kVRounds;
  static_assert(kK8Rounds * NT * 16 == kBlock * D, "INT8 tile must split evenly over the workgroup");
  uint64_t k8src;
  uint32_t k8lds, lane_bytes;
  Kv kv;

  __device__ __forceinline__ Q8Refill(const int8_t* k8tile, uint32_t dst_lds, int wave, int lane, const Kv& v)
      : k8src(uniform64(reinterpret_cast<uint64_t>(k8tile) + uint64_t(wave) * (kWave * 16))),
        k8lds(uint32_t(__builtin_amdgcn_readfirstlane(dst_lds + uint32_t(wave) * (kWave * 16)))),
        lane_bytes(uint32_t(lane) * 16u), kv(v) {}

  __device__ __forceinline__ void round(int r) const {
    if (r < kK8Rounds) {
      uint32_t off = uint32_t(r) * (NT * 16);
      asm volatile("" : "+s"(off));
      dma16(k8src + off, lane_bytes, k8lds + off);
    } else {
      kv.round(r - kK8Rounds + kVRounds);
    }
  }
  __device__ __forceinline__ void all() const {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) round(r);
  }
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

// Materialises a value at this point of the instruction stream, so that the
// work producing it stays ahead of a following branch (where the scheduler
// can overlap it with matrix-core work) instead of being sunk past it.
template <typename T>
__device__ __forceinline__ void pin(T& x) {
  asm volatile("" : "+v"(x));
}

// acc *= alpha, in place (the accumulator keeps its registers on both sides
// of the rare rescale branch instead of being copied).
template <int D>
__device__ __forceinline__ void rescale_acc(State<D>& st, float alpha) {
#pragma unroll
  for (int dt = 0; dt < Shape<D>::DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(st.acc[dt][e]) : "v"(alpha));
}

// Lazy online softmax: the running max m (log2 units, per query) moves only
// when some query's max exceeds it by more than kRescaleSlack.  Otherwise the
// probabilities exp2(s c - m) may exceed 1 by up to 2^kRescaleSlack, which
// FP32 sums and BF16 products carry at unchanged relative precision; acc and
// den always share m, so O = acc / den is unaffected.  The common case has
// no data-dependent branch, so a half's softmax can be spread between
// matrix-core instructions.
constexpr float kRescaleSlack = 8.f;

// Softmax of one 32-key half of raw scores s (absent keys -inf; c = scale *
// log2(e)), in 8 stages that a caller places between MFMAs: max; the
// wave-uniform rescale decision, new max and alpha; 4 x 4 probabilities
// exp2(s c - m); BF16 packing; den update.  The caller multiplies acc by
// alpha when `rescale` is set.
template <int D>
struct HalfSoftmax {
  f32x16 s;
  float mx, alpha, neg_m, lsum;
  bool rescale;
  bf16x8 pw[2];  // packed BF16 probabilities, keys 0..15 / 16..31 of the half

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
      pw[0] = pack8(s, 0);
      pw[1] = pack8(s, 8);
      pin(pw[0]);
      pin(pw[1]);
    } else {
      st.den = st.den * alpha + lsum;
      pin(st.den);
    }
  }
  // The B operand of the P V product for keys 16 c4 .. 16 c4 + 15 of the half.
  __device__ __forceinline__ bf16x8 pb(int c4) const { return pw[c4]; }
  // Part k of n (n = 4 or 8) of the stages.
  template <int N>
  __device__ __forceinline__ void part(int k, State<D>& st, float c) {
#pragma unroll
    for (int i = k * 8 / N; i < (k + 1) * 8 / N; ++i) stage(i, st, c);
  }
};

// Common case of HalfSoftmax without its max pass: the probabilities
// p = exp2(s c - m) are formed against the running max m as it stands, and
// the row sum tells whether that was what HalfSoftmax would have done.  If
// no lane's sum exceeds 255 (or, before any key, 0), every p is below 2^8,
// i.e. every s c - m < log2(255) < kRescaleSlack, so HalfSoftmax would not
// have moved m and would have formed these same p, den += lsum, with acc
// untouched: the results are bit-identical.  Otherwise `redo` is set (a
// wave-uniform ballot) and the caller re-forms the half's raw scores and
// runs HalfSoftmax on them (resolve).  The stages are:
// 4 x 4 probabilities and the row sum; the redo ballot; BF16 packing; den.
constexpr float kFastSumMax = 255.f;

template <int D>
struct FastHalf {
  f32x16 s;
  float lsum, neg_m, thr;
  bool redo;
  bf16x8 pw[2];

  __device__ __forceinline__ void stage(int k, State<D>& st, float c) {
    if (k < 4) {
      if (k == 0) {
        const bool none = st.m == kNegInf;  // nothing yet: p = exp2(s c), and any key moves m
        neg_m = none ? 0.f : -st.m;
        thr = none ? 0.f : kFastSumMax;
        lsum = 0.f;
      }
#pragma unroll
      for (int e = 4 * k; e < 4 * (k + 1); ++e) {
        const float pe = fast_exp2(fmaf(s[e], c, neg_m));
        s[e] = pe;
        lsum += pe;
      }
    } else if (k == 4) {
      redo = __builtin_amdgcn_ballot_w64(lsum > thr) != 0;
    } else if (k == 5) {
      pw[0] = pack8(s, 0);
      pw[1] = pack8(s, 8);
      pin(pw[0]);
      pin(pw[1]);
    } else if (k == 7) {
      st.den = redo ? st.den : st.den + lsum;
      pin(st.den);
    }
  }
  template <int N>
  __device__ __forceinline__ void part(int k, State<D>& st, float c) {
#pragma unroll
    for (int i = k * 8 / N; i < (k + 1) * 8 / N; ++i) stage(i, st, c);
  }
  __device__ __forceinline__ bf16x8 pb(int c4) const { return pw[c4]; }
  // The uncommon case: raw() re-forms the half's scores, HalfSoftmax runs
  // on them (max, rescale decision, probabilities, den), and acc is rescaled
  // if it moved m.
  template <typename Raw>
  __device__ __forceinline__ void resolve(State<D>& st, float c, Raw raw) {
    if (redo) {
      HalfSoftmax<D> full;
      full.s = raw();
#pragma unroll
      for (int i = 0; i < 8; ++i) full.stage(i, st, c);
      if (full.rescale) rescale_acc<D>(st, full.alpha);
      pw[0] = full.pw[0];
      pw[1] = full.pw[1];
    }
  }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));

// This lane's offsets of its MFMA operand reads inside a K + V tile pair
// (TileLayout).  K fragment (t, ks): key row 32 t + col, features
// 16 ks + 8 hh .. +7, at element k_row + 32 t D + (k_x ^ 16 ks).  V^T
// fragment (t, c4, dt): feature 32 dt + col and the 8 keys
// 32 t + 16 c4 + 4 hh + {0..3} and {8..11} (the k-slot order of the score
// result that P^T keeps), as two ds_read_b64_tr_b16.  A transpose read
// hands lane 4 a + e of each 16-lane group element e of the 8-byte reads of
// lanes a, a + 4, a + 8, a + 12, so lane j of the group reads key row
// k0 + (j >> 2), features 4 (j & 3) .. +3 of its 16-feature group: in the
// row-quad V layout that is byte v_lane = 2 (kElems + 8 (hh 4 CPR +
// 4 ((col >> 2) & 3) + 2 (col >> 4) + ((col & 3) >> 1)) + 4 (col & 1)) of
// the tile, and read (t, c4, dt) adds the immediate 64 CPR (8 t + 4 c4) +
// 256 dt bytes (quads of 64 CPR bytes; its second half two quads on).
template <int D>
struct FragLane {
  static constexpr int CPR = TileLayout<D>::kRowChunks;
  int k_row, k_x;
  uint32_t v_lane;
  __device__ __forceinline__ FragLane(int col, int hh)
      : k_row(col * D), k_x(TileLayout<D>::k_lane_xor(col, hh)), v_lane(v_lane_bytes(col, hh)) {}
  __device__ static __forceinline__ uint32_t v_lane_bytes(int col, int hh) {
    const int chunk = hh * 4 * CPR + 4 * ((col >> 2) & 3) + 2 * (col >> 4) + ((col & 3) >> 1);
    return uint32_t(2 * (TileLayout<D>::kElems + 8 * chunk + 4 * (col & 1)));
  }
  __device__ __forceinline__ u32x4 k(const uint16_t* buf, int t, int ks) const {
    return *reinterpret_cast<const u32x4*>(buf + k_row + 32 * t * D + (k_x ^ (16 * ks)));
  }
  // LDS byte address of this lane's V reads in the tile at buf.
  __device__ __forceinline__ uint32_t v_base(const uint16_t* buf) const { return lds_address(buf) + v_lane; }
  __device__ __forceinline__ u32x4 v(uint32_t vbase, int t, int c4, int dt) const {
    const uint32_t a = vbase + uint32_t(64 * CPR * (8 * t + 4 * c4) + 256 * dt);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((SOL_LDS i16x4*)(uintptr_t)a);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((SOL_LDS i16x4*)(uintptr_t)(a + 128u * CPR));
    const u32x2 x = __builtin_bit_cast(u32x2, lo), y = __builtin_bit_cast(u32x2, hi);
    const u32x4 r = {x[0], x[1], y[0], y[1]};
    return r;
  }
};

// Ends a scheduling chunk: nothing moves across it, so the hand-placed
// interleave of matrix-core, LDS, DMA and VALU work below is kept.
__device__ __forceinline__ void chunk_end() { __builtin_amdgcn_sched_barrier(0); }

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

// Barrier that publishes this workgroup's LDS accesses (no global-memory
// fence, so the ring's DMA in flight is not drained).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Bits i of a 64-bit word with lo <= i < hi (any lo, hi).
__device__ __forceinline__ uint64_t bit_range64(int lo, int hi) {
  lo = max(lo, 0);
  hi = min(hi, 64);
  if (hi <= lo) return 0ull;
  const uint64_t upto = hi == 64 ? ~0ull : ((1ull << hi) - 1ull);
  return upto & ~((1ull << lo) - 1ull);
}

// Approximated blocks of centroid tile ct for one query block: blocks of the
// range [lo, hi) whose routing bit is clear.
__device__ __forceinline__ uint64_t tile_approx(const uint32_t* mask, int ct, int lo, int hi) {
  const uint64_t valid = bit_range64(lo - 64 * ct, hi - 64 * ct);
  const uint64_t sel = uint64_t(mask[2 * ct]) | (uint64_t(mask[2 * ct + 1]) << 32);
  return valid & ~sel;
}


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

}  // namespace

}  // namespace sol
