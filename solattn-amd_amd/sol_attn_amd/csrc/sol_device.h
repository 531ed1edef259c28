// Device-side building blocks shared by the SOL routed-attention kernels.
//
// Target: gfx950 (CDNA4), 64-wide wavefronts, bf16 MFMA 32x32x16.
//
// Matrix-core conventions used throughout (v_mfma_f32_32x32x16_bf16):
//   A operand (32 x 16): lane l supplies row (l % 32), k-slots 8*(l/32) .. +7
//   B operand (16 x 32): lane l supplies column (l % 32), k-slots 8*(l/32) .. +7
//   C/D (32 x 32):       lane l holds column (l % 32); element e holds row
//                        8*(e/4) + 4*(l/32) + (e%4)
// Scores are computed transposed, S^T = K * Q^T, so each lane owns ONE query
// (its C column) and the softmax row statistics never leave the lane pair
// (l, l ^ 32).  P^T then feeds O^T = V^T * P^T as the B operand straight
// from registers; the V^T operand is read from row-major V tiles with the
// LDS transpose read ds_read_b64_tr_b16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sol {

constexpr int kBlock = 64;      // tokens per physical block (kernels.py:12)
constexpr int kWave = 64;       // CDNA wavefront width
constexpr int kMaxKeyBlocks = 8192;  // LDS routing bitmask capacity: key blocks routed per segment
constexpr int kPoolChunk = 16;  // key blocks per pooling workgroup (= cascade chunk)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> two round-to-nearest-even bf16 in one v_cvt_pk_bf16_f32
// (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// 32x32x32 INT8 products, INT32 accumulation.  Operand lane layout as the
// BF16 32x32x16 form, with 16 INT8 k-slots per lane (k-slots 16 (l / 32) ..
// +15); the C/D layout is the same.
__device__ __forceinline__ i32x16 mfma32x32x32i8(i32x4 a, i32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 u) { return __builtin_bit_cast(bf16x8, u); }

__device__ __forceinline__ u32x4 zero_u32x4() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

// Row of one attention operand: token t of batch b, head h.  Either strided
// BTHD addressing or (indexed windows) a gather through an int64 token index.
// An index entry outside [0, N) (a plan whose index tensors were changed
// after validation) is clamped into the source, so that every gather stays
// inside the caller's tensor whatever the index holds.
struct TokenRows {
  const uint16_t* base;
  const int64_t* index;  // nullable; [B, T] original token ids
  int64_t sb, st, sh;    // element strides (batch ignored when indexed)
  int64_t N;             // rows an index entry may address (indexed sources)
  int T;

  __device__ __forceinline__ int64_t clamp_row(int64_t r) const { return min(max(r, int64_t(0)), N - 1); }
  __device__ __forceinline__ const uint16_t* row(int b, int t, int h) const {
    if (index) return base + clamp_row(index[int64_t(b) * T + t]) * st + int64_t(h) * sh;
    return base + int64_t(b) * sb + int64_t(t) * st + int64_t(h) * sh;
  }
};

// Operand rows live in global memory: loads through a global-space pointer
// are global_load (vector memory counter only), not flat loads that also
// count against the LDS counter.
typedef const u32x4 __attribute__((address_space(1)))* global_u32x4_ptr;

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *(global_u32x4_ptr)(p);
}

// 16 bytes at element offset `col` of rows t0 .. t0 + N - 1 of entry b, head
// h; rows past t_last (a valid row) read as zero.  The addresses are formed
// first (the index entries of an indexed source all in flight together) and
// every data load is then issued unconditionally -- rows past t_last re-read
// row t_last -- so the N loads are in flight at once instead of each waiting
// behind a branch.  STREAM marks the loads non-temporal (data read once).
template <int N, bool STREAM = false>
__device__ __forceinline__ void load_rows16(const TokenRows& r, int b, int t0, int t_last, int h, int col,
                                            u32x4 (&x)[N]) {
  const uint16_t* p[N];
  if (r.index) {
    const int64_t* idx = r.index + int64_t(b) * r.T;
    int64_t row[N];
#pragma unroll
    for (int i = 0; i < N; ++i) row[i] = r.clamp_row(idx[min(t0 + i, t_last)]);
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = r.base + row[i] * r.st + int64_t(h) * r.sh + col;
  } else {
    const uint16_t* base = r.base + int64_t(b) * r.sb + int64_t(h) * r.sh + col;
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = base + int64_t(min(t0 + i, t_last)) * r.st;
  }
#pragma unroll
  for (int i = 0; i < N; ++i)
    x[i] = STREAM ? __builtin_nontemporal_load((global_u32x4_ptr)(p[i])) : load16(p[i]);
#pragma unroll
  for (int i = 0; i < N; ++i)
    if (t0 + i > t_last) x[i] = zero_u32x4();
}

__device__ __forceinline__ u32x2 load8(const uint16_t* p) {
  return *reinterpret_cast<const u32x2*>(p);
}

// Key-block tiles as the attention kernels hold them in LDS (and as the
// pooling pass writes the centroid tiles and, for indexed windows, the
// gathered key blocks): per key block a K tile then a V tile, 64 key rows x D
// BF16 features each, in 16-byte chunks (8 features) placed so that the MFMA
// operand reads hit distinct LDS banks (64 banks of 4 bytes):
//   K: row-major; chunk c of row r sits at chunk c ^ s_k(r) of the row,
//      s_k(r) = r & 15 for 256-byte rows (D = 128) and (r >> 1) & 7 for
//      128-byte rows (D = 64): the 16 rows of one 16-lane ds_read_b128
//      phase (a score operand) cover all banks.
//   V: row quads; the 4 rows 4 q .. 4 q + 3 fill chunks 4 q CPR ..
//      4 (q + 1) CPR (CPR = D / 8 chunks per row) ordered (c >> 2, r & 3,
//      c & 3).  The P V operand (32 features x 8 keys per lane) is read with
//      ds_read_b64_tr_b16, which gives a lane 4 consecutive keys of one
//      feature: one 32-lane half of a read takes the 4 rows of one quad at
//      4 chunks each, 256 contiguous bytes (all 64 banks), and every part of
//      the address but the lane's own is an immediate.
// Keys past the end of the sequence are zero in the tiles the pooling pass
// writes; kernels that DMA key rows straight from the caller's tensors repeat
// the last valid row there (and mask those keys out of the softmax).
template <int D>
struct TileLayout {
  static constexpr int kElems = kBlock * D;  // elements of one K (or V) tile
  static constexpr int kRowChunks = D / 8;
  __device__ static __forceinline__ int k_swizzle(int row) { return D == 128 ? (row & 15) : ((row >> 1) & 7); }
  // Element offsets (inside the K tile, and inside the V tile) of chunk c of row r.
  __device__ static __forceinline__ int k_offset(int row, int chunk) { return row * D + 8 * (chunk ^ k_swizzle(row)); }
  __device__ static __forceinline__ int v_offset(int row, int chunk) {
    return 8 * ((row >> 2) * 4 * kRowChunks + (chunk >> 2) * 16 + (row & 3) * 4 + (chunk & 3));
  }
  // The score operand read as (lane part) + (XOR part ^ per-read constant):
  // for key row r = 32 t + col and chunk c = 2 ks + hh,
  //   k_offset(r, c) = r D + (k_lane_xor(col, hh) ^ 16 ks),
  // since s_k depends only on col and 2 ks leaves bit 0 free.
  __device__ static __forceinline__ int k_lane_xor(int col, int hh) { return 8 * (hh ^ k_swizzle(col)); }
};

// INT8 K tiles of the quantised-QK experiment: per key block 64 rows x D
// bytes; 16-byte chunk c (features 16 c .. 16 c + 15) of row r sits at chunk
// c ^ s8(r), s8(r) = (r >> 1) & 7 for 128-byte rows (D = 128) and (r >> 2) & 3
// for 64-byte rows (D = 64): the 16 rows of one ds_read_b128 phase then cover
// all 64 banks.  One FP32 scale per block: K = scale * K8.
template <int D>
struct K8Layout {
  static constexpr int kBytes = kBlock * D;
  __device__ static __forceinline__ int swizzle(int row) { return D == 128 ? ((row >> 1) & 7) : ((row >> 2) & 3); }
  __device__ static __forceinline__ int offset(int row, int chunk) { return row * D + 16 * (chunk ^ swizzle(row)); }
};

}  // namespace sol
