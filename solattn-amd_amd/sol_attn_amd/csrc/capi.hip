// extern "C" entry points: argument checks, parameter packing, launches.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "sol_attn_amd.h"
#include "sol_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* msg) {
  g_last_error = msg;
  return code;
}

int hip_status(hipError_t err) {
  if (err == hipSuccess) return SOL_OK;
  g_last_error = std::string("HIP launch failed: ") + hipGetErrorString(err);
  return int(err);
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks one BF16 operand's base pointer and {batch, token, head} strides.
bool operand_ok(const void* base, const int64_t* strides, bool indexed) {
  if (!base || !strides || !aligned16(base)) return false;
  for (int i = 0; i < 3; ++i) {
    if (i == 0 && indexed) continue;
    if (strides[i] <= 0 || strides[i] % 8 != 0) return false;
  }
  return true;
}

bool shape_ok(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim) {
  return batch > 0 && tokens > 0 && heads > 0 && (head_dim == 64 || head_dim == 128) &&
         batch * heads < (int64_t(1) << 24) && tokens < (int64_t(1) << 30);
}

// `rows`: rows an index entry may address (indexed sources; clamped into it).
sol::TokenRows rows_of(const void* base, const int64_t* strides, const int64_t* index, int64_t tokens,
                       int64_t rows = 1) {
  sol::TokenRows r;
  r.base = static_cast<const uint16_t*>(base);
  r.index = index;
  r.N = rows;
  r.sb = strides[0];
  r.st = strides[1];
  r.sh = strides[2];
  r.T = int(tokens);
  return r;
}

// Workspace of sol_attention_noalloc: the pooled key buffers live in this
// file-scope device array instead of caller or library allocations.  Each GPU
// holds its own copy until the process ends.  Host code never passes the
// array's name to a kernel: it passes the per-device address that
// hipGetSymbolAddress returns (scratch_on_current_device).
__device__ __align__(256) uint8_t scratch[SOL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device.
int scratch_on_current_device(void** ptr) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err);
  if (dev < 0 || dev >= kMaxDevices) return fail(SOL_ERR_UNSUPPORTED, "sol_attention_noalloc: device index too large");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_status(err);
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return SOL_OK;
}

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// Routing masks of sol_attention_fwd: uint32 [batch, heads, NQB, ceil(NKB / 32)].
// Tile order of sol_attention_fwd's route workspace (after the masks): int32
// [batch, heads, NQB].
int64_t route_order_bytes(int64_t batch, int64_t query_tokens, int64_t heads) {
  return batch * heads * cdiv(query_tokens, SOL_BLOCK) * 4;
}

int64_t route_mask_bytes(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads) {
  return batch * heads * cdiv(query_tokens, SOL_BLOCK) * cdiv(cdiv(key_tokens, SOL_BLOCK), 32) * 4;
}

// Key-range parts per query-sink tile of the SOL kernel (sol_task).  A
// query-sink block selects every key block, so its workgroup streams all of
// them and, in a launch of few workgroups, ends long after the rest.  Split:
// launches of one-block workgroups (fewer than 512 query-block pairs over all
// (entry, head) pairs, the default schedule's threshold) at finite beta, and
// at beta = +inf (every other workgroup streams its protected blocks only)
// launches of up to 8,192 query blocks (8 rounds of 512 two-block
// workgroups).  Parts hold at least 16 key blocks, at most 8 parts, while
// their partial states fit kSplitBytesMax.  Measured (us per call, 4 heads,
// beta 1): 4,096 tokens 97 -> 60, 8,192 tokens 172 -> 108; at 2 x 4,096 x 16
// heads beta +inf 109 -> 91, while beta 0 or 1 there gains nothing (the
// launch is bound by its two rounds of workgroups, and the extra
// workgroups and the merge cost 1-4%).  beta = -inf (every block exact),
// fewer than two sink blocks and sinks over a quarter of the query blocks
// are not split.
constexpr int64_t kSplitBytesMax = int64_t(64) << 20;

int64_t split_bytes(int64_t bh, int64_t q_sink_blocks, int64_t splits, int64_t head_dim) {
  // Split tiles hold sink blocks [0, 2 floor(q_sink_blocks / 2)) (sink_split_tiles).
  return splits > 1 ? bh * (q_sink_blocks / 2 * 2) * SOL_BLOCK * splits * (head_dim + 4) * 4 : 0;
}

int sink_splits(int64_t bh, int64_t nqb, int64_t nkb, int64_t q_sink_blocks, int force, int64_t head_dim) {
  const bool one_block_groups = bh * ((nqb + 1) / 2) < 512;
  // Launches of the small kernel split every query block's chain inside its
  // workgroup instead.
  if (sol::small_key_split(bh * nqb, nkb, head_dim)) return 1;
  if (force == 1 || q_sink_blocks < 2 || 4 * q_sink_blocks > nqb || nkb > sol::kMaxKeyBlocks ||
      !(one_block_groups || (force == 2 && bh * nqb <= 8192)))
    return 1;
  int64_t s = std::min<int64_t>(8, nkb / 16);
  while (s > 1 && split_bytes(bh, q_sink_blocks, s, head_dim) > kSplitBytesMax) --s;
  return int(std::max<int64_t>(s, 1));
}

// Whether a launch of these sizes over plain K / V rows runs as one kernel
// that pools the keys itself (sol_attention_pools_keys).  Head_dim 64 only:
// every workgroup reads its head's whole K and V to pool them, which the
// four two-wave groups at head_dim 64 absorb (1,024 tokens x 8 heads: 19.1
// us against 23.3 for the pooling kernel + small kernel); at head_dim 128
// the two groups read twice the bytes and lose (33.3 against 24.6 us at
// 1,024 tokens x 4 heads).
bool pools_keys(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads, int64_t head_dim) {
  const int64_t nkb = cdiv(key_tokens, SOL_BLOCK);
  return head_dim == 64 && key_tokens >= SOL_BLOCK && nkb <= sol::kPoolChunk &&
         sol::small_key_split(batch * heads * cdiv(query_tokens, SOL_BLOCK), nkb, head_dim) > 0;
}

int64_t sink_blocks(int64_t query_sink_tokens) {
  const int64_t big = int64_t(1) << 30;
  return cdiv(query_sink_tokens > big ? big : query_sink_tokens, SOL_BLOCK);
}

// Attention kernels DMA key blocks straight from K / V rows ("rows mode",
// no pooled tiles) when the keys are plain strided rows of equal length, at
// least one block of them, with row strides whose 64-row spans fit the
// kernels' 32-bit lane offsets.
bool rows_mode_possible(const int64_t* key_index, const int32_t* key_lengths, int64_t key_tokens,
                        const int64_t* k_strides, const int64_t* v_strides) {
  return !key_index && !key_lengths && key_tokens >= SOL_BLOCK && k_strides && v_strides &&
         k_strides[1] < (int64_t(1) << 24) && v_strides[1] < (int64_t(1) << 24);
}

int rows_mode_ok(const char* who, const void* k, const int64_t* k_strides, const void* v,
                 const int64_t* v_strides, const int32_t* key_lengths, int64_t key_tokens) {
  static thread_local std::string msg;
  if (!operand_ok(k, k_strides, false) || !operand_ok(v, v_strides, false) ||
      !rows_mode_possible(nullptr, key_lengths, key_tokens, k_strides, v_strides)) {
    msg = std::string(who) +
          ": without tiles, K and V must be 16-byte aligned strided rows (token stride < 2^24 elements), "
          "key_lengths NULL and key_tokens >= 64";
    return fail(SOL_ERR_INVALID, msg.c_str());
  }
  return SOL_OK;
}

// Checks of the attention launch shared by sol_attention_fwd and
// sol_attention_noalloc (which runs them before its pooling launch, so that a
// rejected call launches nothing).
int attention_args_ok(const char* who, const void* q, const int64_t* q_strides, bool indexed, int64_t batch,
                      int64_t query_tokens, int64_t heads, double scale, double beta, int64_t kv_sink_tokens,
                      int64_t query_sink_tokens, const void* out) {
  static thread_local std::string msg;
  const char* what = nullptr;
  if (!operand_ok(q, q_strides, indexed))
    what = ": Q needs 16-byte aligned rows and positive strides";
  else if (!std::isfinite(scale) || scale <= 0)
    what = ": scale must be finite and positive";
  else if (std::isnan(beta))
    what = ": beta must not be NaN";
  else if (kv_sink_tokens < 0 || query_sink_tokens < 0)
    what = ": sink token counts must be nonnegative";
  else if (!out || !aligned16(out))
    what = ": out must be a 16-byte aligned device buffer";
  if (what) {
    msg = std::string(who) + what;
    return fail(SOL_ERR_INVALID, msg.c_str());
  }
  if (batch * heads * cdiv(query_tokens, SOL_BLOCK) >= (int64_t(1) << 31)) {
    msg = std::string(who) + ": grid too large";
    return fail(SOL_ERR_UNSUPPORTED, msg.c_str());
  }
  return SOL_OK;
}

// sol_attention_fwd with, at finite beta, the pooling pass's chunk sums in
// place of key_mean / key_var (chunk_sums non-null: the cutoff stage folds
// the moments itself; folds_moments key sequences, no key_lengths, no
// route_workspace or key_cov).
int attention_fwd_impl(const void* q, const int64_t* q_strides, const int64_t* query_index,
                      int64_t sequence_length, int64_t batch, int64_t query_tokens,
                      int64_t key_tokens,
                      const int32_t* key_lengths, int64_t heads, int64_t head_dim,
                      const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      const void* tiles, const void* ctiles, const float* key_mean,
                      const float* key_var, const float* key_cov, const uint8_t* protection,
                      const int32_t* pair_strides, void* split_workspace, void* route_workspace,
                      const float* query_means, double scale, double beta,
                      int64_t local_blocks, int64_t kv_sink_tokens, int64_t query_sink_tokens,
                      void* out, const int64_t* out_index, int32_t* counts,
                      uint8_t* debug_selected, float* debug_proxy, float* debug_cutoff,
                      const void* qk_int8_tiles, const float* qk_int8_scales,
                      int workgroup_form, void* stream,
                       const float* chunk_sums, bool tile_moments);

}  // namespace

extern "C" {

int sol_abi_version(void) { return SOL_ABI_VERSION; }

const char* sol_last_error(void) { return g_last_error.c_str(); }

int sol_pool_sizes(int64_t batch, int64_t key_tokens, int64_t heads, int64_t head_dim,
                   int64_t sizes[4]) {
  if (!sizes || !shape_ok(batch, key_tokens, heads, head_dim))
    return fail(SOL_ERR_INVALID, "sol_pool_sizes: invalid shape");
  const int64_t nkb = cdiv(key_tokens, SOL_BLOCK);
  const int64_t nct = cdiv(nkb, SOL_BLOCK);
  const int64_t tile = 2 * SOL_BLOCK * head_dim * 2;
  sizes[0] = batch * heads * nct * tile;
  sizes[1] = batch * heads * nkb * tile;
  sizes[2] = batch * heads * cdiv(nkb, 16) * 2 * head_dim * 4;
  sizes[3] = batch * heads * head_dim * 4;
  return SOL_OK;
}

namespace {

int pool_checked(const char* who, const void* k, const int64_t* k_strides, const void* v,
                 const int64_t* v_strides, const int64_t* key_index, const int32_t* key_lengths,
                 int64_t sequence_length, int64_t batch, int64_t key_tokens, int64_t heads,
                 int64_t head_dim, void* ctiles, void* tiles,
                 float* chunk_sums, float* key_mean, float* key_var, void* stream,
                 bool fold_in_attention = false, bool blocks_only = false) {
  static thread_local std::string msg;
  auto err = [&](int code, const char* what) {
    msg = std::string(who) + ": " + what;
    return fail(code, msg.c_str());
  };
  if (!shape_ok(batch, key_tokens, heads, head_dim))
    return err(SOL_ERR_INVALID, "unsupported shape (head_dim must be 64 or 128)");
  const bool indexed = key_index != nullptr;
  if (!operand_ok(k, k_strides, indexed) || !operand_ok(v, v_strides, indexed))
    return err(SOL_ERR_INVALID, "K/V need 16-byte aligned rows and positive strides");
  if (indexed && sequence_length <= 0)
    return err(SOL_ERR_INVALID, "an indexed source needs sequence_length > 0");
  if (!ctiles && !tiles) return err(SOL_ERR_INVALID, "nothing to write");
  if ((ctiles && !aligned16(ctiles)) || (tiles && !aligned16(tiles)))
    return err(SOL_ERR_INVALID, "ctiles/tiles must be 16-byte aligned device buffers");
  const bool moments = chunk_sums || key_mean || key_var;
  if (moments && !(chunk_sums && key_mean && key_var && ctiles))
    return err(SOL_ERR_INVALID, "chunk_sums, key_mean and key_var go together (with ctiles)");
  const int64_t nkb = cdiv(key_tokens, SOL_BLOCK);
  if (key_tokens > SOL_MAX_KEY_TOKENS) return err(SOL_ERR_UNSUPPORTED, "key_tokens exceeds SOL_MAX_KEY_TOKENS");
  sol::PoolParams p{};
  p.k = rows_of(k, k_strides, key_index, key_tokens, sequence_length);
  p.v = rows_of(v, v_strides, key_index, key_tokens, sequence_length);
  p.klen = key_lengths;
  p.ctiles = static_cast<uint16_t*>(ctiles);
  p.tiles = static_cast<uint16_t*>(tiles);
  p.ksum = moments ? chunk_sums : nullptr;
  p.mean = key_mean;
  p.var = key_var;
  p.B = int(batch);
  p.H = int(heads);
  p.Tk = int(key_tokens);
  p.NKB = int(nkb);
  p.NCT = int(cdiv(nkb, SOL_BLOCK));
  p.NCHP = p.NCT * (SOL_BLOCK / sol::kPoolChunk);
  p.fold_in_attention = fold_in_attention ? 1 : 0;
  // Centroid tiles only (all_in): plain rows, at most 16 blocks, nothing else.
  if (blocks_only && (tiles || !ctiles || key_index || key_lengths || moments || nkb > sol::kPoolChunk))
    return err(SOL_ERR_INVALID, "centroid-only pooling needs plain rows, ctiles only and at most 16 key blocks");
  p.blocks_only = blocks_only ? 1 : 0;
  return hip_status(sol::launch_pool(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

}  // namespace

int sol_pool_kv(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                const int64_t* key_index, const int32_t* key_lengths, int64_t sequence_length,
                int64_t batch, int64_t key_tokens, int64_t heads, int64_t head_dim, void* ctiles,
                void* tiles, float* chunk_sums, float* key_mean, float* key_var, void* stream) {
  return pool_checked("sol_pool_kv", k, k_strides, v, v_strides, key_index, key_lengths,
                      sequence_length, batch, key_tokens, heads, head_dim, ctiles, tiles,
                      chunk_sums, key_mean, key_var, stream);
}

int64_t sol_pair_workspace_size(int64_t batch, int64_t query_tokens, int64_t heads, int64_t head_dim) {
  if (!shape_ok(batch, query_tokens, heads, head_dim)) return 0;
  const int64_t nqb = cdiv(query_tokens, SOL_BLOCK);
  if (nqb < 4 || nqb > sol::kMaxPairBlocks) return 0;
  return batch * heads * head_dim * (nqb + sol::kMaxLag) * int64_t(sizeof(float));
}

int sol_pair_strides(const void* q, const int64_t* q_strides, const int64_t* query_index,
                     int64_t sequence_length, int64_t batch, int64_t query_tokens,
                     int64_t heads, int64_t head_dim, void* workspace, int32_t* strides,
                     float* query_means, void* stream) {
  const int64_t bytes = sol_pair_workspace_size(batch, query_tokens, heads, head_dim);
  if (bytes == 0)
    return fail(SOL_ERR_UNSUPPORTED,
                "sol_pair_strides: needs 4 .. 8192 query blocks and head_dim 64 or 128");
  if (!operand_ok(q, q_strides, query_index != nullptr))
    return fail(SOL_ERR_INVALID, "sol_pair_strides: Q needs 16-byte aligned rows and positive strides");
  if (!workspace || !strides || !aligned16(workspace))
    return fail(SOL_ERR_INVALID, "sol_pair_strides: workspace (16-byte aligned) and strides are required");
  if (query_index && sequence_length <= 0)
    return fail(SOL_ERR_INVALID, "sol_pair_strides: an indexed Q needs sequence_length > 0");
  sol::PairParams p{};
  p.q = rows_of(q, q_strides, query_index, query_tokens, sequence_length);
  p.B = int(batch);
  p.H = int(heads);
  p.Tq = int(query_tokens);
  p.NQB = int(cdiv(query_tokens, SOL_BLOCK));
  p.means = static_cast<float*>(workspace);
  p.lags = p.means + batch * heads * head_dim * p.NQB;
  p.strides = strides;
  p.qc = query_means;
  return hip_status(sol::launch_pairing(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

int sol_plan_protection(const int64_t* rows, const int64_t* keys, const int32_t* key_lengths,
                        int64_t windows, int64_t query_rows, int64_t key_count,
                        int64_t local_tokens, const int64_t* ranges, int64_t nranges,
                        uint8_t* protected_blocks, void* stream) {
  if (windows <= 0 || query_rows <= 0 || key_count <= 0 || local_tokens < 0 || nranges < 0 ||
      nranges > (int64_t(1) << 20) || query_rows >= (int64_t(1) << 40) || key_count >= (int64_t(1) << 40))
    return fail(SOL_ERR_INVALID, "sol_plan_protection: invalid shape or range count");
  if (!rows || !keys || !protected_blocks || (nranges > 0 && !ranges))
    return fail(SOL_ERR_INVALID, "sol_plan_protection: rows, keys, ranges and protected_blocks are required");
  sol::PlanParams p{};
  p.rows = rows;
  p.keys = keys;
  p.key_lengths = key_lengths;
  p.ranges = ranges;
  p.out = protected_blocks;
  p.W = windows;
  p.nq = query_rows;
  p.nk = key_count;
  p.NQB = cdiv(query_rows, SOL_BLOCK);
  p.NKB = cdiv(key_count, SOL_BLOCK);
  p.local = local_tokens;
  p.nranges = int(nranges);
  if (p.W * p.NQB * p.NKB >= (int64_t(1) << 38))  // grid of < 2^30 workgroups
    return fail(SOL_ERR_INVALID, "sol_plan_protection: plan too large");
  return hip_status(sol::launch_plan_protection(p, static_cast<hipStream_t>(stream)));
}

int64_t sol_key_covariance_workspace_size(int64_t batch, int64_t heads, int64_t head_dim) {
  if (!shape_ok(batch, 1, heads, head_dim)) return 0;
  return batch * heads * sol::kCovSplit * head_dim * head_dim * 4;
}

int sol_key_covariance(const void* ctiles, const float* key_mean, const int32_t* key_lengths,
                       int64_t batch, int64_t key_tokens, int64_t heads, int64_t head_dim,
                       void* workspace, float* key_cov, void* stream) {
  if (!shape_ok(batch, key_tokens, heads, head_dim))
    return fail(SOL_ERR_INVALID, "sol_key_covariance: invalid shape");
  if (!ctiles || !aligned16(ctiles) || !key_mean || !workspace || !key_cov)
    return fail(SOL_ERR_INVALID, "sol_key_covariance: ctiles (16-byte aligned), key_mean, workspace and key_cov are required");
  const int64_t nkb = cdiv(key_tokens, SOL_BLOCK);
  sol::CovParams p{};
  p.ctiles = static_cast<const uint16_t*>(ctiles);
  p.mean = key_mean;
  p.klen = key_lengths;
  p.partial = static_cast<float*>(workspace);
  p.cov = key_cov;
  p.B = int(batch);
  p.H = int(heads);
  p.Tk = int(key_tokens);
  p.NCT = int(cdiv(nkb, SOL_BLOCK));
  return hip_status(sol::launch_covariance(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

int64_t sol_split_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                                 int64_t head_dim, double beta, int64_t query_sink_tokens) {
  if (!shape_ok(batch, query_tokens, heads, head_dim) || key_tokens <= 0 || key_tokens >= (int64_t(1) << 30) ||
      query_sink_tokens < 0 || std::isnan(beta))
    return 0;
  const int64_t bh = batch * heads, nqb = cdiv(query_tokens, SOL_BLOCK), qsb = sink_blocks(query_sink_tokens);
  const int force = std::isinf(beta) ? (beta < 0 ? 1 : 2) : 0;
  const int s = sink_splits(bh, nqb, cdiv(key_tokens, SOL_BLOCK), qsb, force, head_dim);
  return split_bytes(bh, qsb, s, head_dim);
}

int64_t sol_route_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                                 double beta) {
  if (!shape_ok(batch, query_tokens, heads, 64) || key_tokens <= 0 || key_tokens >= (int64_t(1) << 30) ||
      std::isnan(beta))
    return 0;
  if (std::isinf(beta) && beta < 0) return 0;  // every block exact: no routing
  return align256(route_mask_bytes(batch, query_tokens, key_tokens, heads)) + route_order_bytes(batch, query_tokens, heads);
}

int sol_attention_pools_keys(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                             int64_t head_dim) {
  return shape_ok(batch, query_tokens, heads, head_dim) && key_tokens > 0 && key_tokens < (int64_t(1) << 30) &&
                 pools_keys(batch, query_tokens, key_tokens, heads, head_dim)
             ? 1 : 0;
}

int sol_attention_fwd(const void* q, const int64_t* q_strides, const int64_t* query_index,
                      int64_t sequence_length, int64_t batch, int64_t query_tokens,
                      int64_t key_tokens,
                      const int32_t* key_lengths, int64_t heads, int64_t head_dim,
                      const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      const void* tiles, const void* ctiles, const float* key_mean,
                      const float* key_var, const float* key_cov, const uint8_t* protection,
                      const int32_t* pair_strides, void* split_workspace, void* route_workspace,
                      const float* query_means, double scale, double beta,
                      int64_t local_blocks, int64_t kv_sink_tokens, int64_t query_sink_tokens,
                      void* out, const int64_t* out_index, int32_t* counts,
                      uint8_t* debug_selected, float* debug_proxy, float* debug_cutoff,
                      const void* qk_int8_tiles, const float* qk_int8_scales,
                      int workgroup_form, void* stream) {
  return attention_fwd_impl(q, q_strides, query_index, sequence_length, batch, query_tokens, key_tokens,
                            key_lengths, heads, head_dim, k, k_strides, v, v_strides, tiles, ctiles, key_mean,
                            key_var, key_cov, protection, pair_strides, split_workspace, route_workspace,
                            query_means, scale, beta, local_blocks, kv_sink_tokens, query_sink_tokens, out,
                            out_index, counts, debug_selected, debug_proxy, debug_cutoff, qk_int8_tiles,
                            qk_int8_scales, workgroup_form, stream, nullptr, false);
}

int sol_quantize_keys(const void* k, const int64_t* k_strides, const int64_t* key_index,
                      const int32_t* key_lengths, int64_t sequence_length, int64_t batch, int64_t key_tokens,
                      int64_t heads, int64_t head_dim, int rows_mode, void* k8_tiles, float* k8_scales,
                      void* stream) {
  if (!shape_ok(batch, key_tokens, heads, head_dim))
    return fail(SOL_ERR_INVALID, "sol_quantize_keys: unsupported shape (head_dim must be 64 or 128)");
  if (!operand_ok(k, k_strides, key_index != nullptr))
    return fail(SOL_ERR_INVALID, "sol_quantize_keys: K needs 16-byte aligned rows and positive strides");
  if (key_index && sequence_length <= 0)
    return fail(SOL_ERR_INVALID, "sol_quantize_keys: an indexed source needs sequence_length > 0");
  if (!k8_tiles || !k8_scales || !aligned16(k8_tiles))
    return fail(SOL_ERR_INVALID, "sol_quantize_keys: k8_tiles (16-byte aligned) and k8_scales are required");
  if (rows_mode && (key_index || key_lengths || key_tokens < SOL_BLOCK))
    return fail(SOL_ERR_INVALID, "sol_quantize_keys: rows_mode needs plain K rows (no index, no key_lengths) "
                                 "and key_tokens >= 64");
  const int64_t ntiles = batch * heads * cdiv(key_tokens, SOL_BLOCK);
  if (ntiles >= (int64_t(1) << 31)) return fail(SOL_ERR_UNSUPPORTED, "sol_quantize_keys: grid too large");
  sol::QuantParams p{};
  p.k = rows_of(k, k_strides, key_index, key_tokens, sequence_length);
  p.klen = key_lengths;
  p.k8 = static_cast<int8_t*>(k8_tiles);
  p.scale = k8_scales;
  p.B = int(batch);
  p.H = int(heads);
  p.Tk = int(key_tokens);
  p.NKB = int(cdiv(key_tokens, SOL_BLOCK));
  p.shifted = rows_mode ? 1 : 0;
  return hip_status(sol::launch_quantize_keys(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

int sol_dense_fwd(const void* q, const int64_t* q_strides, const int64_t* query_index, int64_t sequence_length,
                  const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                  int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                  int64_t head_dim, double scale, void* tiles, void* out, const int64_t* out_index,
                  void* stream) {
  if (!shape_ok(batch, query_tokens, heads, head_dim) || key_tokens <= 0 ||
      key_tokens >= (int64_t(1) << 30))
    return fail(SOL_ERR_INVALID, "sol_dense_fwd: unsupported shape (head_dim must be 64 or 128)");
  if (!operand_ok(q, q_strides, query_index != nullptr))
    return fail(SOL_ERR_INVALID, "sol_dense_fwd: Q needs 16-byte aligned rows and positive strides");
  if ((query_index || out_index) && sequence_length <= 0)
    return fail(SOL_ERR_INVALID, "sol_dense_fwd: query_index / out_index need sequence_length > 0");
  if (!std::isfinite(scale) || scale <= 0)
    return fail(SOL_ERR_INVALID, "sol_dense_fwd: scale must be finite and positive");
  if (!out || !aligned16(out)) return fail(SOL_ERR_INVALID, "sol_dense_fwd: out must be 16-byte aligned");
  if (batch * heads * cdiv(query_tokens, 128) >= (int64_t(1) << 31))
    return fail(SOL_ERR_UNSUPPORTED, "sol_dense_fwd: grid too large");
  // Key blocks straight from K / V rows, or (fewer than 64 keys, or token
  // strides too large for rows mode) from tiles pooled into the workspace.
  const bool rows = rows_mode_possible(nullptr, nullptr, key_tokens, k_strides, v_strides);
  if (rows) {
    const int rc = rows_mode_ok("sol_dense_fwd", k, k_strides, v, v_strides, nullptr, key_tokens);
    if (rc != SOL_OK) return rc;
  } else {
    if (!tiles) return fail(SOL_ERR_INVALID, "sol_dense_fwd: this shape needs the tiles workspace");
    const int rc = pool_checked("sol_dense_fwd", k, k_strides, v, v_strides, nullptr, nullptr, 0, batch,
                                key_tokens, heads, head_dim, nullptr, tiles, nullptr, nullptr,
                                nullptr, stream);
    if (rc != SOL_OK) return rc;
  }
  sol::AttnParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = rows_of(q, q_strides, query_index, query_tokens, sequence_length);
  p.out_index = out_index;
  p.out_rows = sequence_length;
  p.tiles = rows ? nullptr : static_cast<const uint16_t*>(tiles);
  if (rows) {
    p.k = rows_of(k, k_strides, nullptr, key_tokens);
    p.v = rows_of(v, v_strides, nullptr, key_tokens);
  }
  p.out = static_cast<uint16_t*>(out);
  p.B = int(batch);
  p.H = int(heads);
  p.Tq = int(query_tokens);
  p.Tk = int(key_tokens);
  p.NQB = int(cdiv(query_tokens, SOL_BLOCK));
  p.NKB = int(cdiv(key_tokens, SOL_BLOCK));
  p.scale = float(scale);
  p.scale_log2 = float(scale * 1.4426950408889634);
  return hip_status(sol::launch_dense(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace {

int attention_fwd_impl(const void* q, const int64_t* q_strides, const int64_t* query_index,
                      int64_t sequence_length, int64_t batch, int64_t query_tokens,
                      int64_t key_tokens,
                      const int32_t* key_lengths, int64_t heads, int64_t head_dim,
                      const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      const void* tiles, const void* ctiles, const float* key_mean,
                      const float* key_var, const float* key_cov, const uint8_t* protection,
                      const int32_t* pair_strides, void* split_workspace, void* route_workspace,
                      const float* query_means, double scale, double beta,
                      int64_t local_blocks, int64_t kv_sink_tokens, int64_t query_sink_tokens,
                      void* out, const int64_t* out_index, int32_t* counts,
                      uint8_t* debug_selected, float* debug_proxy, float* debug_cutoff,
                      const void* qk_int8_tiles, const float* qk_int8_scales,
                      int workgroup_form, void* stream,
                       const float* chunk_sums, bool tile_moments) {
  if (!shape_ok(batch, query_tokens, heads, head_dim) || key_tokens <= 0 ||
      key_tokens >= (int64_t(1) << 30))
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: unsupported shape (head_dim must be 64 or 128)");
  const int arc = attention_args_ok("sol_attention_fwd", q, q_strides, query_index != nullptr, batch,
                                    query_tokens, heads, scale, beta, kv_sink_tokens, query_sink_tokens, out);
  if (arc != SOL_OK) return arc;
  if ((query_index || out_index) && sequence_length <= 0)
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: query_index / out_index need sequence_length > 0");
  if (workgroup_form < 0 || workgroup_form > 2)
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: workgroup_form must be 0, 1 or 2");
  if ((qk_int8_tiles == nullptr) != (qk_int8_scales == nullptr) || (qk_int8_tiles && !aligned16(qk_int8_tiles)))
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: qk_int8_tiles (16-byte aligned) and qk_int8_scales go together");
  const int force = std::isinf(beta) ? (beta < 0 ? 1 : 2) : 0;
  // Without centroid tiles the launch pools the keys itself (or, at beta =
  // -inf, needs none).
  const bool self_pooled = !ctiles && force != 1;
  if (self_pooled && (tiles || key_lengths || query_index || key_cov || qk_int8_tiles || route_workspace ||
                      workgroup_form != 0 || !pools_keys(batch, query_tokens, key_tokens, heads, head_dim)))
    return fail(SOL_ERR_INVALID,
                "sol_attention_fwd: ctiles may be NULL only at beta = -inf or where sol_attention_pools_keys "
                "holds (plain K / V rows, no key_lengths, query_index, key_cov, INT8 tiles or route_workspace, "
                "workgroup_form 0)");
  if ((ctiles && !aligned16(ctiles)) || (tiles && !aligned16(tiles)) ||
      (split_workspace && !aligned16(split_workspace)) || (route_workspace && !aligned16(route_workspace)))
    return fail(SOL_ERR_INVALID,
                "sol_attention_fwd: tiles/ctiles/split_workspace/route_workspace must be 16-byte aligned "
                "device buffers");
  if (query_means && !route_workspace)
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: query_means are read only with a route_workspace");
  if (!tiles) {
    const int rc = rows_mode_ok("sol_attention_fwd", k, k_strides, v, v_strides, key_lengths, key_tokens);
    if (rc != SOL_OK) return rc;
  }
  if (chunk_sums && (force != 0 || self_pooled || key_lengths || route_workspace || key_cov ||
                     !sol::folds_moments(cdiv(key_tokens, SOL_BLOCK))))
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: chunk sums in place of the moments need finite beta, "
                                 "17..255 key blocks, no key_lengths, route_workspace or key_cov");
  if (tile_moments && (force != 0 || self_pooled || chunk_sums || key_lengths || route_workspace || key_cov ||
                       !ctiles || cdiv(key_tokens, SOL_BLOCK) > sol::kPoolChunk))
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: moments from the centroid tile need finite beta, "
                                 "ctiles, at most 16 key blocks, no key_lengths, route_workspace or key_cov");
  if (force == 0 && !self_pooled && !chunk_sums && !tile_moments && (!key_mean || !key_var))
    return fail(SOL_ERR_INVALID, "sol_attention_fwd: finite beta needs key_mean and key_var");
  const int64_t nkb = cdiv(key_tokens, SOL_BLOCK);
  const int64_t nqb = cdiv(query_tokens, SOL_BLOCK);
  sol::AttnParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = rows_of(q, q_strides, query_index, query_tokens, sequence_length);
  p.pair_stride = pair_strides;
  p.klen = key_lengths;
  p.out_index = out_index;
  p.out_rows = sequence_length;
  p.workgroup_form = workgroup_form;
  p.k8 = static_cast<const int8_t*>(qk_int8_tiles);
  p.k8_scale = qk_int8_scales;
  p.tiles = static_cast<const uint16_t*>(tiles);
  if (!tiles) {
    p.k = rows_of(k, k_strides, nullptr, key_tokens);
    p.v = rows_of(v, v_strides, nullptr, key_tokens);
  }
  p.ctiles = static_cast<const uint16_t*>(ctiles);
  p.mean = chunk_sums || tile_moments ? nullptr : key_mean;
  p.var = chunk_sums || tile_moments ? nullptr : key_var;
  p.ksum = chunk_sums;
  p.tile_moments = tile_moments ? 1 : 0;
  p.cov = force == 0 ? key_cov : nullptr;
  p.protection = protection;
  p.out = static_cast<uint16_t*>(out);
  p.counts = counts;
  p.dbg_selected = debug_selected;
  p.dbg_proxy = debug_proxy;
  p.dbg_cutoff = debug_cutoff;
  p.B = int(batch);
  p.H = int(heads);
  p.Tq = int(query_tokens);
  p.Tk = int(key_tokens);
  p.NQB = int(nqb);
  p.NKB = int(nkb);
  p.NCT = int(cdiv(nkb, SOL_BLOCK));
  p.scale = float(scale);
  p.scale_log2 = float(scale * 1.4426950408889634);
  p.beta = force == 0 ? float(beta) : 0.f;
  p.force = force;
  const int64_t big = int64_t(1) << 30;
  p.local_blocks = int(local_blocks < 0 ? -1 : (local_blocks > big ? big : local_blocks));
  p.kv_sink_blocks = int(cdiv(kv_sink_tokens > big ? big : kv_sink_tokens, SOL_BLOCK));
  p.q_sink_blocks = int(sink_blocks(query_sink_tokens));
  p.splits = split_workspace ? sink_splits(batch * heads, nqb, nkb, p.q_sink_blocks, force, head_dim) : 1;
  p.partial = p.splits > 1 ? static_cast<float*>(split_workspace) : nullptr;
  p.mask = force != 1 ? static_cast<uint32_t*>(route_workspace) : nullptr;
  p.order = p.mask ? reinterpret_cast<int32_t*>(static_cast<uint8_t*>(route_workspace) +
                                                align256(route_mask_bytes(batch, query_tokens, key_tokens, heads)))
                   : nullptr;
  p.NW = int(cdiv(nkb, 32));
  p.qc = query_means;
  return hip_status(sol::launch_sol(p, int(head_dim), static_cast<hipStream_t>(stream)));
}

// Byte layout of the all-in workspace: the sol_pool_kv buffers, 256-byte
// aligned, in the order sol_pool_sizes lists them (the block tiles only
// outside rows mode, the moment buffers only at finite beta), then the split
// workspace.  total 0: the launch pools its keys itself and needs none.
struct AllInLayout {
  bool rows, moments, self_pooled;
  int64_t tiles, sums, mean, var, split, split_bytes, total;
};

AllInLayout all_in_layout(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                          int64_t head_dim, double beta, int64_t query_sink_tokens, bool rows) {
  AllInLayout l{};
  l.rows = rows;
  l.moments = std::isfinite(beta);
  l.self_pooled = rows && !(std::isinf(beta) && beta < 0) &&
                  pools_keys(batch, query_tokens, key_tokens, heads, head_dim);
  if (l.self_pooled) return l;
  int64_t sizes[4];
  sol_pool_sizes(batch, key_tokens, heads, head_dim, sizes);
  l.tiles = align256(sizes[0]);
  l.sums = l.tiles + (rows ? 0 : align256(sizes[1]));
  l.mean = l.sums + align256(sizes[2]);
  l.var = l.mean + align256(sizes[3]);
  l.split = l.moments ? l.var + align256(sizes[3]) : l.sums;
  l.split_bytes = sol_split_workspace_size(batch, query_tokens, key_tokens, heads, head_dim, beta,
                                           query_sink_tokens);
  l.total = l.split + align256(l.split_bytes);
  return l;
}

// Pooling + attention over BTHD inputs in workspace `ws` (`ws_bytes` bytes;
// NULL / 0 when the launch pools its keys itself).  `scratch`: the workspace
// is the library's device array (sol_attention_noalloc), looked up only after
// every check has passed, and `ws` is ignored.
int all_in(const char* who, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
           const void* v, const int64_t* v_strides, int64_t batch, int64_t query_tokens, int64_t key_tokens,
           int64_t heads, int64_t head_dim, double scale, double beta, int64_t local_blocks,
           int64_t kv_sink_tokens, int64_t query_sink_tokens, uint8_t* ws, int64_t ws_bytes, bool scratch,
           void* out, int32_t* counts, void* stream) {
  static thread_local std::string msg;
  if (!shape_ok(batch, query_tokens, heads, head_dim) || !shape_ok(batch, key_tokens, heads, head_dim) ||
      key_tokens >= (int64_t(1) << 30)) {
    msg = std::string(who) + ": unsupported shape (head_dim must be 64 or 128)";
    return fail(SOL_ERR_INVALID, msg.c_str());
  }
  const int arc = attention_args_ok(who, q, q_strides, false, batch, query_tokens, heads, scale, beta,
                                    kv_sink_tokens, query_sink_tokens, out);
  if (arc != SOL_OK) return arc;
  const bool rows = rows_mode_possible(nullptr, nullptr, key_tokens, k_strides, v_strides);
  const AllInLayout l = all_in_layout(batch, query_tokens, key_tokens, heads, head_dim, beta, query_sink_tokens,
                                      rows);
  // One attention launch that pools the keys itself: no workspace at all.
  if (l.self_pooled)
    return sol_attention_fwd(q, q_strides, nullptr, 0, batch, query_tokens, key_tokens, nullptr, heads, head_dim,
                             k, k_strides, v, v_strides, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr, nullptr, nullptr, scale, beta, local_blocks, kv_sink_tokens,
                             query_sink_tokens, out, nullptr, counts, nullptr, nullptr, nullptr, nullptr, nullptr,
                             0, stream);
  if (l.total > ws_bytes) {
    msg = scratch ? std::string(who) +
                        ": the pooled keys need more than SOL_NOALLOC_SCRATCH_BYTES (128 MiB); use "
                        "sol_attention_all_in or sol_pool_kv + sol_attention_fwd with caller workspace"
                  : std::string(who) + ": workspace_bytes is below sol_attention_workspace_size";
    return fail(scratch ? SOL_ERR_UNSUPPORTED : SOL_ERR_INVALID, msg.c_str());
  }
  if (scratch) {
    void* base = nullptr;
    const int rc = scratch_on_current_device(&base);
    if (rc != SOL_OK) return rc;
    ws = static_cast<uint8_t*>(base);
  } else if (!aligned16(ws)) {
    msg = std::string(who) + ": workspace must be a 16-byte aligned device buffer";
    return fail(SOL_ERR_INVALID, msg.c_str());
  }
  float* sums = l.moments ? reinterpret_cast<float*>(ws + l.sums) : nullptr;
  float* mean = l.moments ? reinterpret_cast<float*>(ws + l.mean) : nullptr;
  float* var = l.moments ? reinterpret_cast<float*>(ws + l.var) : nullptr;
  void* tiles = rows ? nullptr : ws + l.tiles;
  // Moments of 17..255 key blocks: the attention workgroups fold the chunk
  // sums themselves (the same bits) and the moments_kernel launch goes.
  // All-in calls, one box, alternating libraries, us: 4,096 tokens x 4 heads
  // 44.3 -> 43.4, 8,192 x 4 70.9 -> 70.1, 4,096 x 16 73.5 -> 71.3; 2 x 4,096
  // x 16 163.1 -> 162.1 and 4,096 x 10,000 keys x 24 heads 235.3 -> 233.8
  // (with the fold's loads issued together, before the query mean).
  const bool fold = l.moments && sol::folds_moments(cdiv(key_tokens, SOL_BLOCK));
  // Keys of at most one 16-block chunk in rows mode: the centroid tiles alone
  // (pool_blocks_kernel, 16 workgroups per head instead of one per head and
  // K / V), and the attention launch forms the moments from tile 0.
  const bool blocks = rows && cdiv(key_tokens, SOL_BLOCK) <= sol::kPoolChunk;
  const bool tile_moments = blocks && l.moments;
  const int prc = blocks ? pool_checked(who, k, k_strides, v, v_strides, nullptr, nullptr, 0, batch, key_tokens,
                                        heads, head_dim, ws, nullptr, nullptr, nullptr, nullptr, stream, false, true)
                         : pool_checked(who, k, k_strides, v, v_strides, nullptr, nullptr, 0, batch, key_tokens,
                                        heads, head_dim, ws, tiles, sums, mean, var, stream, fold);
  if (prc != SOL_OK) return prc;
  return attention_fwd_impl(q, q_strides, nullptr, 0, batch, query_tokens, key_tokens, nullptr, heads,
                            head_dim, k, k_strides, v, v_strides, tiles, ws, mean, var, nullptr, nullptr, nullptr,
                            l.split_bytes ? ws + l.split : nullptr, nullptr /* routing in the attention kernel */,
                            nullptr, scale, beta, local_blocks, kv_sink_tokens, query_sink_tokens, out, nullptr,
                            counts, nullptr, nullptr, nullptr, nullptr, nullptr, 0, stream, fold ? sums : nullptr,
                            tile_moments);
}

}  // namespace

extern "C" {

int64_t sol_attention_workspace_size(int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                                     int64_t head_dim, double beta, int64_t query_sink_tokens,
                                     int64_t k_token_stride, int64_t v_token_stride) {
  if (!shape_ok(batch, query_tokens, heads, head_dim) || !shape_ok(batch, key_tokens, heads, head_dim) ||
      key_tokens >= (int64_t(1) << 30) || query_sink_tokens < 0 || std::isnan(beta) || k_token_stride <= 0 ||
      v_token_stride <= 0)
    return -1;
  const int64_t ks[3] = {0, k_token_stride, 1}, vs[3] = {0, v_token_stride, 1};
  const bool rows = rows_mode_possible(nullptr, nullptr, key_tokens, ks, vs);
  return all_in_layout(batch, query_tokens, key_tokens, heads, head_dim, beta, query_sink_tokens, rows).total;
}

int sol_attention_all_in(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, int64_t batch, int64_t query_tokens,
                         int64_t key_tokens, int64_t heads, int64_t head_dim, double scale, double beta,
                         int64_t local_blocks, int64_t kv_sink_tokens, int64_t query_sink_tokens, void* workspace,
                         int64_t workspace_bytes, void* out, int32_t* counts, void* stream) {
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(SOL_ERR_INVALID, "sol_attention_all_in: workspace_bytes must be >= 0, with a workspace if > 0");
  return all_in("sol_attention_all_in", q, q_strides, k, k_strides, v, v_strides, batch, query_tokens, key_tokens,
                heads, head_dim, scale, beta, local_blocks, kv_sink_tokens, query_sink_tokens,
                static_cast<uint8_t*>(workspace), workspace_bytes, false, out, counts, stream);
}

int sol_attention_noalloc(const void* q, const int64_t* q_strides, const void* k,
                          const int64_t* k_strides, const void* v, const int64_t* v_strides,
                          int64_t batch, int64_t query_tokens, int64_t key_tokens, int64_t heads,
                          int64_t head_dim, double scale, double beta, int64_t local_blocks,
                          int64_t kv_sink_tokens, int64_t query_sink_tokens, void* out,
                          int32_t* counts, void* stream) {
  return all_in("sol_attention_noalloc", q, q_strides, k, k_strides, v, v_strides, batch, query_tokens, key_tokens,
                heads, head_dim, scale, beta, local_blocks, kv_sink_tokens, query_sink_tokens, nullptr,
                SOL_NOALLOC_SCRATCH_BYTES, true, out, counts, stream);
}

}  // extern "C"
