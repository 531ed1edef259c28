// Fused SOL routing + attention, and the dense flash-attention control, for gfx950.
//
// Replaces the reference's `_threshold` (src/sol_attn_amd/kernels.py:52-64),
// `_sol` (kernels.py:101-182) and `_dense` (kernels.py:67-98).
//
// One SOL workgroup = one 64-query block of one (batch, head): 2 waves, each
// owning 32 queries.  Phases:
//   1. stage the Q tile in LDS; Q^T fragments go to registers (MFMA B operand)
//   2. FP32 query mean (torch cascade order) and the Eq.15 cutoff
//      c = Qc.mu + beta * sqrt(sum Qc^2 var)            (kernels.py:58-63)
//   3. routing: proxy_j = Qc . Kc_j (the mean over the block's rows of
//      q_r . Kc_j), selected = proxy > c, OR sink / local / plan protection;
//      decisions live in an LDS bitmask, never in HBM      (kernels.py:129-143)
//   4. centroid correction for unselected blocks, 32 centroids per MFMA tile:
//      w = exp2(s - m) * valid_len, O^T += Vc^T * bf16(w)^T (kernels.py:145-158)
//   5. exact blocks in ascending order from the bitmask: K / V^T tiles in LDS,
//      S^T = K Q^T, online softmax, O^T += V^T * bf16(P)^T (kernels.py:159-178)
//   6. O = acc / den, BF16 store; exact-block count       (kernels.py:179-182)
// All contributions share one FP32 online-softmax state per query, kept in
// log2 units.  The dense control runs phase 5 over every key block with
// 128 queries per workgroup.
#include "sol_device.h"
#include "sol_internal.h"

namespace sol {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// Maps the linear workgroup id so that every XCD (ids are dealt round-robin
// over the 8 XCDs) receives a contiguous range of tasks: neighbouring query
// blocks of one head then share that XCD's L2.
__device__ __forceinline__ int xcd_task(int i, int n) {
  const int xcd = i & 7, slot = i >> 3;
  const int per = n >> 3, rem = n & 7;
  return xcd * per + min(xcd, rem) + slot;
}

template <int D>
struct Tile {
  static constexpr int KS = D + 8;      // K / Q row stride (elements), 16B rows
  static constexpr int VS = kBlock + 4; // V^T row stride (elements)
  static constexpr int DC = D / 8;      // 16-byte chunks per row
  static constexpr int KT = D / 16;     // MFMA k-steps over the head dimension
  static constexpr int DT = D / 32;     // 32-wide output tiles over the head dimension
  static constexpr int KV_ELEMS = kBlock * KS + D * VS;
};

// Per-lane online-softmax state: one query per lane, shared by lanes l, l^32.
template <int D>
struct SoftmaxState {
  f32x16 acc[Tile<D>::DT];
  float m;    // running max (log2 units), -inf until the first contribution
  float den;  // this lane's partial denominator (its 16 of each 32 keys)
};

template <int D>
__device__ __forceinline__ void load_kv_tile(const AttnParams& p, int b, int h, int j,
                                             uint16_t* sk, uint16_t* svt, int tid, int nt) {
  using T = Tile<D>;
  const int t0 = j * kBlock;
  for (int idx = tid; idx < kBlock * T::DC; idx += nt) {
    const int r = idx / T::DC, c = idx % T::DC;
    const int t = t0 + r;
    const u32x4 x = t < p.Tk ? load16(p.k.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(sk + r * T::KS + 8 * c) = x;
  }
  for (int idx = tid; idx < 8 * T::DC; idx += nt) {
    const int g = (idx & 3) + 4 * (idx / (4 * T::DC));  // 8-key group
    const int c = (idx >> 2) % T::DC;                   // 8-feature chunk
    u32x4 rows[8], cols[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = t0 + 8 * g + i;
      rows[i] = t < p.Tk ? load16(p.v.row(b, t, h) + 8 * c) : zero_u32x4();
    }
    transpose8x8(rows, cols);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u32x2* dst = reinterpret_cast<u32x2*>(svt + (8 * c + i) * T::VS + 8 * g);
      dst[0] = u32x2{cols[i][0], cols[i][1]};
      dst[1] = u32x2{cols[i][2], cols[i][3]};
    }
  }
}

// One exact 64-key block from LDS into the softmax state.
template <int D>
__device__ __forceinline__ void exact_block(const AttnParams& p, int j, const bf16x8 (&qf)[Tile<D>::KT],
                                            const uint16_t* sk, const uint16_t* svt, int col, int hh,
                                            SoftmaxState<D>& st) {
  using T = Tile<D>;
  f32x16 s[2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    s[kt] = zero16();
#pragma unroll
    for (int ks = 0; ks < T::KT; ++ks) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(sk + (kt * 32 + col) * T::KS + ks * 16 + 8 * hh);
      s[kt] = mfma32x32x16(as_bf16x8(a), qf[ks], s[kt]);
    }
  }
  const int key0 = j * kBlock + 4 * hh;
  const bool tail = (j + 1) * kBlock > p.Tk;
  float mx = kNegInf;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = s[kt][e] * p.scale_log2;
      if (tail && key0 + kt * 32 + 8 * (e >> 2) + (e & 3) >= p.Tk) v = kNegInf;
      s[kt][e] = v;
      mx = fmaxf(mx, v);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mnew = fmaxf(st.m, mx);
  const float alpha = fast_exp2(st.m - mnew);
  float lsum = 0.f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = fast_exp2(s[kt][e] - mnew);
      s[kt][e] = pe;
      lsum += pe;
    }
  }
  st.den = st.den * alpha + lsum;
  st.m = mnew;
#pragma unroll
  for (int dt = 0; dt < T::DT; ++dt) st.acc[dt] *= alpha;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pb[i] = pack_bf16x2(s[c >> 1][8 * (c & 1) + 2 * i], s[c >> 1][8 * (c & 1) + 2 * i + 1]);
    const bf16x8 b = as_bf16x8(pb);
#pragma unroll
    for (int dt = 0; dt < T::DT; ++dt) {
      const uint16_t* row = svt + (dt * 32 + col) * T::VS + 16 * c + 4 * hh;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(row);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(row + 8);
      const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
      st.acc[dt] = mfma32x32x16(as_bf16x8(a), b, st.acc[dt]);
    }
  }
}

template <int D>
__device__ __forceinline__ void store_output(const AttnParams& p, int b, int h, int t,
                                             int hh, const SoftmaxState<D>& st) {
  using T = Tile<D>;
  const float den = st.den + __shfl_xor(st.den, 32);
  if (t >= p.Tq) return;
  uint16_t* orow = p.out + ((int64_t(b) * p.Tq + t) * p.H + h) * D;
#pragma unroll
  for (int dt = 0; dt < T::DT; ++dt) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      u32x2 o;
      o[0] = pack_bf16x2(__fdiv_rn(st.acc[dt][4 * k4], den), __fdiv_rn(st.acc[dt][4 * k4 + 1], den));
      o[1] = pack_bf16x2(__fdiv_rn(st.acc[dt][4 * k4 + 2], den), __fdiv_rn(st.acc[dt][4 * k4 + 3], den));
      *reinterpret_cast<u32x2*>(orow + dt * 32 + 8 * k4 + 4 * hh) = o;
    }
  }
}

}  // namespace

template <int D, int NW, bool SOL>
__global__ __launch_bounds__(NW * 64) void attention_kernel(AttnParams p) {
  using T = Tile<D>;
  constexpr int NT = NW * 64;
  constexpr int QROWS = NW * 32;
  constexpr int Q_ELEMS = QROWS * T::KS;
  constexpr int U_ELEMS = Q_ELEMS > T::KV_ELEMS ? Q_ELEMS : T::KV_ELEMS;
  __shared__ __align__(16) uint16_t su[U_ELEMS];   // Q staging, then K / V^T tiles
  __shared__ float s_qm[D];
  __shared__ float s_red[2 * NW];
  __shared__ uint32_t s_mask[SOL ? kMaxKeyBlocks / 32 : 1];
  uint16_t* sk = su;
  uint16_t* svt = su + kBlock * T::KS;

  const int nq_tiles = (p.Tq + QROWS - 1) / QROWS;
  const int task = xcd_task(blockIdx.x, gridDim.x);
  const int qt = task % nq_tiles;
  const int bh = task / nq_tiles;
  const int h = bh % p.H, b = bh / p.H;
  const int q0 = qt * QROWS;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, hh = lane >> 5;

  // 1. Q tile -> LDS -> register fragments.
  for (int idx = tid; idx < QROWS * T::DC; idx += NT) {
    const int r = idx / T::DC, c = idx % T::DC;
    const int t = q0 + r;
    const u32x4 x = t < p.Tq ? load16(p.q.row(b, t, h) + 8 * c) : zero_u32x4();
    *reinterpret_cast<u32x4*>(su + r * T::KS + 8 * c) = x;
  }
  __syncthreads();
  bf16x8 qf[T::KT];
  const int myq = wave * 32 + col;
#pragma unroll
  for (int ks = 0; ks < T::KT; ++ks)
    qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(su + myq * T::KS + ks * 16 + 8 * hh));

  SoftmaxState<D> st;
#pragma unroll
  for (int dt = 0; dt < T::DT; ++dt) st.acc[dt] = zero16();
  st.m = kNegInf;
  st.den = 0.f;

  if constexpr (SOL) {
    const int qb = qt;
    const int64_t head = int64_t(b) * p.H + h;
    float cut = 0.f;
    // 2. Query mean (torch order: 16-row sequential chunks folded in order) and cutoff.
    if (p.force == 0) {
      const int qlen = min(kBlock, p.Tq - q0);
      if (tid < D) {
        float tot = 0.f;
        for (int c = 0; c < 4; ++c) {
          float s = 0.f;
          for (int i = 0; i < 16; ++i) {
            const int r = 16 * c + i;
            if (r < qlen) s = __fadd_rn(s, bf16_bits_to_f32(su[r * T::KS + tid]));
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
        s_red[NW + wave] = g;
      }
      __syncthreads();
      float mu = 0.f, sg = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        mu += s_red[w];
        sg += s_red[NW + w];
      }
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
          for (int c = 0; c < T::DC; ++c) {
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
    if (p.counts && tid == 0) {
      int cnt = 0;
      for (int w = 0; w < nwords; ++w) cnt += __builtin_popcount(s_mask[w]);
      p.counts[(int64_t(b) * p.NQB + qb) * p.H + h] = cnt;
    }

    // 4. Centroid correction for unselected blocks, 32 centroids per tile.
    if (p.force != 1) {
      const uint16_t* kc = p.kc + head * p.NKB * D;
      const uint16_t* vct = p.vct + head * D * p.NKBP;
      for (int t0 = 0; t0 < p.NKB; t0 += 32) {
        const int nvalid = min(32, p.NKB - t0);
        const uint32_t validw = nvalid == 32 ? 0xFFFFFFFFu : ((1u << nvalid) - 1u);
        const uint32_t apw = validw & ~s_mask[t0 >> 5];
        if (apw == 0) continue;
        f32x16 sc = zero16();
        const bool row_ok = t0 + col < p.NKB;
#pragma unroll
        for (int ks = 0; ks < T::KT; ++ks) {
          const u32x4 a = row_ok ? load16(kc + int64_t(t0 + col) * D + ks * 16 + 8 * hh) : zero_u32x4();
          sc = mfma32x32x16(as_bf16x8(a), qf[ks], sc);
        }
        float mx = kNegInf;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
          const float v = ((apw >> r) & 1u) ? sc[e] * p.scale_log2 : kNegInf;
          sc[e] = v;
          mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(st.m, mx);
        const float safe = mnew == kNegInf ? 0.f : mnew;
        const float alpha = fast_exp2(st.m - safe);
        float lsum = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = 8 * (e >> 2) + 4 * hh + (e & 3);
          float w = 0.f;
          if ((apw >> r) & 1u) {
            const float len = float(min(kBlock, p.Tk - kBlock * (t0 + r)));
            w = fast_exp2(sc[e] - safe) * len;
          }
          sc[e] = w;
          lsum += w;
        }
        st.den = st.den * alpha + lsum;
        st.m = mnew;
#pragma unroll
        for (int dt = 0; dt < T::DT; ++dt) st.acc[dt] *= alpha;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          u32x4 pb;
#pragma unroll
          for (int i = 0; i < 4; ++i) pb[i] = pack_bf16x2(sc[8 * c + 2 * i], sc[8 * c + 2 * i + 1]);
          const bf16x8 bw = as_bf16x8(pb);
#pragma unroll
          for (int dt = 0; dt < T::DT; ++dt) {
            const uint16_t* row = vct + int64_t(dt * 32 + col) * p.NKBP + t0 + 16 * c + 4 * hh;
            const u32x2 lo = load8(row);
            const u32x2 hi = load8(row + 8);
            const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
            st.acc[dt] = mfma32x32x16(as_bf16x8(a), bw, st.acc[dt]);
          }
        }
      }
    }

    // 5. Exact blocks, ascending.
    for (int w = 0; w < nwords; ++w) {
      uint32_t bits = s_mask[w];
      while (bits) {
        const int j = w * 32 + __builtin_ctz(bits);
        bits &= bits - 1u;
        __syncthreads();
        load_kv_tile<D>(p, b, h, j, sk, svt, tid, NT);
        __syncthreads();
        exact_block<D>(p, j, qf, sk, svt, col, hh, st);
      }
    }
  } else {
    for (int j = 0; j < p.NKB; ++j) {
      __syncthreads();
      load_kv_tile<D>(p, b, h, j, sk, svt, tid, NT);
      __syncthreads();
      exact_block<D>(p, j, qf, sk, svt, col, hh, st);
    }
  }

  // 6. Normalise and store.
  store_output<D>(p, b, h, q0 + myq, hh, st);
}

hipError_t launch_sol(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned grid = unsigned(p.B) * p.H * p.NQB;
  if (D == 128)
    hipLaunchKernelGGL((attention_kernel<128, 2, true>), dim3(grid), dim3(128), 0, stream, p);
  else
    hipLaunchKernelGGL((attention_kernel<64, 2, true>), dim3(grid), dim3(128), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_dense(const AttnParams& p, int D, hipStream_t stream) {
  const unsigned tiles = unsigned((p.Tq + 127) / 128);
  const unsigned grid = unsigned(p.B) * p.H * tiles;
  if (D == 128)
    hipLaunchKernelGGL((attention_kernel<128, 4, false>), dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((attention_kernel<64, 4, false>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace sol
