// Kernel 1: reshape-and-cache scatter of new K/V rows into pool slots.
//
// Behaviour of PagedKVCachePool.write_prefill (src/mini_infra/worker/paged_kv_cache.py:74-95)
// and of the decode append in Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:282-283),
// as one launch covering every layer instead of an advanced-index gather plus an index_copy_
// per tensor per layer.
//
// Work mapping: a token is one destination K row and one V row of num_kv_heads * head_dim
// elements (2 KiB each for 8 x 128 bf16), contiguous in the pool.
//  * Span kernel (16-byte aligned rows and strides -- every real shape): grid z picks K or V, and
//    a workgroup moves the rows of kSpanTokens consecutive index entries of one layer.  Lane i of a
//    128-lane row team moves 16-byte piece i (+ 128 k) of a token's row, so each wavefront access
//    is one contiguous 1 KiB run of a row.  The (row, position, slot) triples are wave-uniform and
//    read with scalar loads, all before the first data load; every data load of a lane is issued
//    before its first store.
//  * Generic kernel (any other row size or misaligned strides): flat piece index with
//    element-size pieces; used by small shapes only.
//
// XCD runs.  Workgroups are dealt round-robin to the 8 XCDs.  Taken in index order, two tokens
// whose rows share an aligned 4 KiB region of the source or of the pool then land on different
// XCDs, and on MI355X that costs ~3% per side.  The prefill store always has such tokens: prompts
// are left-padded in the source, and each prompt starts on a block boundary in the pool, so the
// two sides' alignments differ per prompt.  The kernel therefore maps blockIdx so that each XCD
// takes runs of kXcdRun consecutive token groups.
//
// Measured on MI355X (28-layer prefill store of 32 prompts U[128, 2048], 40,636 tokens, token-major
// source rows; two repetitions in one process; read + write copy ceiling 6.64-6.72 TB/s, copy into
// 32 KiB units at scattered places 5.63-5.76):
//   form (lanes x tokens per workgroup, store, XCD run)   near-sequential tables   fragmented tables
//   128 x 1, non-temporal, runs of 128                       6.56-6.58 TB/s           5.87-5.88
//   256 x 2 (one token per row team), nt, runs of 64         6.42-6.58                5.80-5.87
//   256 x 2, nt, runs of 128 / 256 / 32 / 16                 6.48-6.55 / 6.49 / 6.40-6.46 / 6.07-6.09
//   256 x 2, device-scope streaming stores, runs of 64       6.36-6.37                5.82-5.84
//   128 x 2 (two tokens per lane), streaming, no runs        6.04-6.22                5.51-5.66
//   the earlier LDS-staged form (K and V together, 2 tokens)  6.11-6.25                5.43-5.59
//   16 tokens (one pool block) per workgroup, 128-1024 lanes 5.34-5.87                5.19-5.48
//   workgroups looping over token groups (grid-stride)       4.99-5.86                4.91-5.79
// Best case for comparison (packed source, identity slots, no runs): 6.50-6.53 TB/s.  Padding the
// index so each contiguous run starts at index = slot (mod 16) adds under 1% and is not done.
#include "mi_common.h"

#ifndef MI_SCATTER_NT
#define MI_SCATTER_NT 1
#endif
#ifndef MI_SCATTER_SPAN_THREADS
#define MI_SCATTER_SPAN_THREADS 128
#endif
#ifndef MI_SCATTER_SPAN_TOKENS
#define MI_SCATTER_SPAN_TOKENS 1
#endif
#ifndef MI_SCATTER_SPLIT_KV
#define MI_SCATTER_SPLIT_KV 1
#endif
#ifndef MI_SCATTER_STREAM
#define MI_SCATTER_STREAM 0
#endif
#ifndef MI_SCATTER_XCD_RUN
#define MI_SCATTER_XCD_RUN 128
#endif
#ifndef MI_SCATTER_NARROW
#define MI_SCATTER_NARROW 1
#endif

namespace mi {
namespace {

constexpr bool kNt = MI_SCATTER_NT != 0;  // non-temporal source loads and pool stores
constexpr int kGenericThreads = 128;
constexpr int kGenericUnroll = 8;
constexpr int kGenericTokensPerGroup = 8;
constexpr int kRowLanes = 128;  // lanes of a row team
constexpr int kSpanThreads = MI_SCATTER_SPAN_THREADS;
constexpr int kSpanTokens = MI_SCATTER_SPAN_TOKENS;
constexpr bool kSplitKv = MI_SCATTER_SPLIT_KV != 0;        // K and V rows in separate workgroups
constexpr bool kStreamStores = MI_SCATTER_STREAM != 0;     // device-scope streaming pool stores
constexpr int kXcdRun = MI_SCATTER_XCD_RUN;                // token groups per XCD run (0: none)
static_assert(kSpanThreads % kRowLanes == 0 && kSpanTokens % (kSpanThreads / kRowLanes) == 0,
              "span kernel: whole row teams, whole tokens per team");

struct ScatterArgs {
  const char* key_src[kMaxLayersPerLaunch];
  const char* value_src[kMaxLayersPerLaunch];
  char* key_pool[kMaxLayersPerLaunch];
  char* value_pool[kMaxLayersPerLaunch];
  const int64_t* token_rows;       // may be null: row i
  const int64_t* token_positions;  // may be null: position 0
  const int64_t* slot_mapping;
  int64_t index_stride;
  int64_t num_tokens;
  int64_t num_slots;
  int64_t num_rows, num_positions;  // source extents along the row and position axes
  // Byte strides of the sources.
  int64_t key_row, key_head, key_pos;
  int64_t value_row, value_head, value_pos;
  uint32_t row_bytes;        // bytes of one pool row (num_kv_heads * head_dim * elem)
  uint32_t head_bytes;       // bytes of one head (head_dim * elem)
  uint32_t chunks_per_head;  // head_bytes / piece
  uint32_t chunks_per_row;   // num_kv_heads * chunks_per_head
  int32_t tokens_per_group;  // span kernel: index entries per workgroup (<= kSpanTokens)
  int64_t groups;            // token groups: ceil(num_tokens / tokens_per_group)
};

// Source byte offsets of token i for K and V; slot -1 when the token is skipped.
struct TokenRef {
  int64_t key_off, value_off, slot;
};

__device__ __forceinline__ TokenRef token_ref(const ScatterArgs& a, int64_t i) {
  const int64_t slot = a.slot_mapping[i * a.index_stride];
  const int64_t row = a.token_rows ? a.token_rows[i * a.index_stride] : i;
  const int64_t pos = a.token_positions ? a.token_positions[i * a.index_stride] : 0;
  const bool ok = slot >= 0 && slot < a.num_slots && row >= 0 && row < a.num_rows && pos >= 0 &&
                  pos < a.num_positions;
  TokenRef t;
  t.slot = ok ? slot : -1;
  t.key_off = row * a.key_row + pos * a.key_pos;
  t.value_off = row * a.value_row + pos * a.value_pos;
  return t;
}

// kNarrow: every source and pool byte offset fits in 32 bits (checked by the host), so offsets are
// formed with 32-bit multiplies.  kRowContig: a token's heads are adjacent in the source (the
// model's token-major K/V rows), so piece p of the row is at byte 16 p.
template <bool kNarrow, bool kRowContig>
__global__ __launch_bounds__(kSpanThreads) void reshape_and_cache_span(const ScatterArgs a) {
  constexpr int kSide = kSpanThreads / kRowLanes;  // row teams (tokens side by side)
  constexpr int kPer = kSpanTokens / kSide;        // tokens per lane
  constexpr int kKv = kSplitKv ? 1 : 2;
  const int layer = blockIdx.y;
  // A row team is two whole wavefronts, so its index is wave-uniform.
  const int team = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kRowLanes);
  const uint32_t lane = threadIdx.x % kRowLanes;
  int64_t g = blockIdx.x;
  if (kXcdRun > 0) {
    // Within each super-run of kXcds * kXcdRun groups, the workgroups that land on XCD x (every
    // kXcds-th) take groups [x kXcdRun, (x + 1) kXcdRun) in order; the partial tail keeps identity.
    constexpr int64_t kSuper = static_cast<int64_t>(kXcds) * kXcdRun;
    if (g < a.groups / kSuper * kSuper) {
      const int64_t base = g / kSuper * kSuper, r = g - base;
      g = base + (r % kXcds) * kXcdRun + r / kXcds;
    }
  }
  const int64_t tok0 = g * a.tokens_per_group;
  const int ntok = static_cast<int>(min(static_cast<int64_t>(a.tokens_per_group), a.num_tokens - tok0));
  // All index loads first (clamped to the group's last entry so every address is valid).
  int64_t slot[kPer], row[kPer], pos[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int64_t i = tok0 + min(team + k * kSide, ntok - 1);
    slot[k] = a.slot_mapping[i * a.index_stride];
    row[k] = a.token_rows ? a.token_rows[i * a.index_stride] : i;
    pos[k] = a.token_positions ? a.token_positions[i * a.index_stride] : 0;
  }
  int64_t src_off[kKv][kPer], dst_off[kPer];
  bool live[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    live[k] = team + k * kSide < ntok && static_cast<uint64_t>(slot[k]) < static_cast<uint64_t>(a.num_slots) &&
              static_cast<uint64_t>(row[k]) < static_cast<uint64_t>(a.num_rows) &&
              static_cast<uint64_t>(pos[k]) < static_cast<uint64_t>(a.num_positions);
    int64_t key_off, value_off;
    if (kNarrow) {
      const uint32_t r = static_cast<uint32_t>(row[k]), q = static_cast<uint32_t>(pos[k]);
      dst_off[k] = static_cast<uint32_t>(slot[k]) * a.row_bytes;
      key_off = r * static_cast<uint32_t>(a.key_row) + q * static_cast<uint32_t>(a.key_pos);
      value_off = r * static_cast<uint32_t>(a.value_row) + q * static_cast<uint32_t>(a.value_pos);
    } else {
      dst_off[k] = slot[k] * a.row_bytes;
      key_off = row[k] * a.key_row + pos[k] * a.key_pos;
      value_off = row[k] * a.value_row + pos[k] * a.value_pos;
    }
    // A skipped token still loads (offset 0 of the source, which the host guarantees is
    // non-empty), so every lane's loads are unconditional and issue back to back; only its stores
    // are skipped.
    if (!live[k]) key_off = value_off = 0;
    if (kSplitKv) {
      src_off[0][k] = blockIdx.z ? value_off : key_off;
    } else {
      src_off[0][k] = key_off;
      src_off[kKv - 1][k] = value_off;
    }
  }
  const char* src_base[kKv];
  char* dst_base[kKv];
#pragma unroll
  for (int kv = 0; kv < kKv; ++kv) {
    const bool is_value = kSplitKv ? blockIdx.z != 0 : kv == 1;
    src_base[kv] = is_value ? a.value_src[layer] : a.key_src[layer];
    dst_base[kv] = is_value ? a.value_pool[layer] : a.key_pool[layer];
  }
  // Passes over the row are uniform (a lane past the row's end loads piece 0 and stores nothing),
  // so the index triples stay in scalar registers.
  const uint32_t passes = (a.chunks_per_row + kRowLanes - 1) / kRowLanes;
  for (uint32_t pass = 0; pass < passes; ++pass) {
    const uint32_t p = lane + pass * kRowLanes;
    const bool in_row = p < a.chunks_per_row;
    const uint32_t pc = in_row ? p : 0u;
    const uint32_t h = kRowContig ? 0u : pc / a.chunks_per_head;
    const uint32_t j = pc - h * a.chunks_per_head;
    u32x4 val[kKv][kPer];
#pragma unroll
    for (int kv = 0; kv < kKv; ++kv) {
      const bool is_value = kSplitKv ? blockIdx.z != 0 : kv == 1;
      const char* src =
          src_base[kv] + (kRowContig ? pc * 16u : h * (is_value ? a.value_head : a.key_head) + j * 16u);
#pragma unroll
      for (int k = 0; k < kPer; ++k) val[kv][k] = load_vec<kNt>(reinterpret_cast<const u32x4*>(src + src_off[kv][k]));
    }
    if (!in_row) continue;
#pragma unroll
    for (int kv = 0; kv < kKv; ++kv)
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        if (!live[k]) continue;
        u32x4* out = reinterpret_cast<u32x4*>(dst_base[kv] + p * 16u + dst_off[k]);
        if (kStreamStores)
          store_stream<kNt>(out, val[kv][k]);
        else
          store_vec<kNt>(out, val[kv][k]);
      }
  }
}

// Generic kernel: flat piece index, any piece size V.
template <typename V>
__global__ __launch_bounds__(kGenericThreads) void reshape_and_cache_generic(const ScatterArgs a) {
  const int layer = blockIdx.y;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * kGenericTokensPerGroup;
  const int64_t ntok = min(static_cast<int64_t>(kGenericTokensPerGroup), a.num_tokens - tok0);
  const uint32_t per_token = 2u * a.chunks_per_row;  // K row then V row
  const uint32_t n_items = static_cast<uint32_t>(ntok) * per_token;

  for (uint32_t base = 0; base < n_items; base += kGenericThreads * kGenericUnroll) {
    V val[kGenericUnroll];
    V* dst[kGenericUnroll];
#pragma unroll
    for (int k = 0; k < kGenericUnroll; ++k) {
      const uint32_t f = base + k * kGenericThreads + threadIdx.x;
      dst[k] = nullptr;
      if (f < n_items) {
        const uint32_t t = f / per_token;
        const uint32_t r = f - t * per_token;
        const TokenRef ref = token_ref(a, tok0 + t);
        if (ref.slot >= 0) {
          const bool is_value = r >= a.chunks_per_row;
          const uint32_t w = is_value ? r - a.chunks_per_row : r;
          const uint32_t h = w / a.chunks_per_head;
          const uint32_t j = w - h * a.chunks_per_head;
          const char* src = is_value ? a.value_src[layer] + ref.value_off + h * a.value_head
                                     : a.key_src[layer] + ref.key_off + h * a.key_head;
          val[k] = *reinterpret_cast<const V*>(src + j * sizeof(V));
          char* pool = is_value ? a.value_pool[layer] : a.key_pool[layer];
          dst[k] = reinterpret_cast<V*>(pool + ref.slot * a.row_bytes + w * sizeof(V));
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kGenericUnroll; ++k)
      if (dst[k]) *dst[k] = val[k];
  }
}

}  // namespace
}  // namespace mi

extern "C" int32_t mi_reshape_and_cache(const void* const* key_src, const void* const* value_src,
                                        int64_t key_row_stride, int64_t key_head_stride, int64_t key_pos_stride,
                                        int64_t value_row_stride, int64_t value_head_stride,
                                        int64_t value_pos_stride, const int64_t* token_rows,
                                        const int64_t* token_positions, const int64_t* slot_mapping,
                                        int64_t index_stride, int64_t num_tokens, int64_t num_src_rows,
                                        int64_t num_src_positions, void* const* key_pools,
                                        void* const* value_pools, int32_t num_layers, int64_t num_slots,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t elem_bytes, void* stream) {
  using namespace mi;
  if (num_tokens < 0 || num_layers < 0 || num_slots < 0 || num_src_rows < 0 || num_src_positions < 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_reshape_and_cache: negative size");
  // With no source rows or positions every token is skipped: nothing to write.
  if (num_tokens == 0 || num_layers == 0 || num_src_rows == 0 || num_src_positions == 0) return ok();
  if (!key_src || !value_src || !key_pools || !value_pools || !slot_mapping)
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_reshape_and_cache: null pointer argument");
  if (num_kv_heads <= 0 || head_dim <= 0 || (elem_bytes != 2 && elem_bytes != 4))
    return fail(MI_ERR_INVALID_ARGUMENT, "mi_reshape_and_cache: bad shape (heads=%d head_dim=%d elem=%d)",
                num_kv_heads, head_dim, elem_bytes);
  if (index_stride <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "mi_reshape_and_cache: index_stride must be > 0");

  ScatterArgs a{};
  a.token_rows = token_rows;
  a.token_positions = token_positions;
  a.slot_mapping = slot_mapping;
  a.index_stride = index_stride;
  a.num_tokens = num_tokens;
  a.num_slots = num_slots;
  a.num_rows = num_src_rows;
  a.num_positions = num_src_positions;
  a.key_row = key_row_stride * elem_bytes;
  a.key_head = key_head_stride * elem_bytes;
  a.key_pos = key_pos_stride * elem_bytes;
  a.value_row = value_row_stride * elem_bytes;
  a.value_head = value_head_stride * elem_bytes;
  a.value_pos = value_pos_stride * elem_bytes;
  a.head_bytes = static_cast<uint32_t>(head_dim) * elem_bytes;
  a.row_bytes = a.head_bytes * num_kv_heads;

  // The widest piece every address is a multiple of: 16 B on the usual
  // contiguous bf16 tensors, else the element size.
  bool wide = a.head_bytes % 16 == 0;
  const int64_t strides[6] = {a.key_row, a.key_head, a.key_pos, a.value_row, a.value_head, a.value_pos};
  for (int64_t s : strides) wide = wide && (s % 16 == 0);
  for (int l = 0; l < num_layers && wide; ++l)
    wide = aligned16(key_src[l]) && aligned16(value_src[l]) && aligned16(key_pools[l]) && aligned16(value_pools[l]);
  const uint32_t piece = wide ? 16u : static_cast<uint32_t>(elem_bytes);
  a.chunks_per_head = a.head_bytes / piece;
  a.chunks_per_row = a.chunks_per_head * num_kv_heads;
  if (2ull * a.chunks_per_row * kGenericTokensPerGroup >= (1ull << 31))
    return fail(MI_ERR_UNSUPPORTED, "mi_reshape_and_cache: row of %u bytes too large", a.row_bytes);
  const bool span_kernel = wide;
  // Few tokens (a decode append) go one per workgroup, spread over the CUs; many tokens (a prompt)
  // go kSpanTokens per workgroup.
  int64_t per_group = kGenericTokensPerGroup;
  if (span_kernel) {
    const int64_t spread = (num_tokens * num_layers + 2047) / 2048;
    per_group = spread < 1 ? 1 : (spread > kSpanTokens ? kSpanTokens : spread);
  }
  a.tokens_per_group = static_cast<int32_t>(per_group);

  const int64_t groups = (num_tokens + per_group - 1) / per_group;
  a.groups = groups;
  const bool row_contig = a.key_head == a.head_bytes && a.value_head == a.head_bytes;
  // 32-bit offsets when every source byte a token can address and every pool byte fits (strides
  // non-negative): the largest row and position, plus the largest head, plus one head.
  bool narrow = MI_SCATTER_NARROW != 0;
  for (int64_t st : strides) narrow = narrow && st >= 0 && st < (int64_t{1} << 32);
  if (narrow) {
    const __int128 last_key = static_cast<__int128>(num_src_rows - 1) * a.key_row +
                              static_cast<__int128>(num_src_positions - 1) * a.key_pos +
                              static_cast<__int128>(num_kv_heads - 1) * a.key_head + a.head_bytes;
    const __int128 last_value = static_cast<__int128>(num_src_rows - 1) * a.value_row +
                                static_cast<__int128>(num_src_positions - 1) * a.value_pos +
                                static_cast<__int128>(num_kv_heads - 1) * a.value_head + a.head_bytes;
    const __int128 pool_bytes = static_cast<__int128>(num_slots) * a.row_bytes;
    const __int128 lim = static_cast<__int128>(1) << 32;
    narrow = last_key <= lim && last_value <= lim && pool_bytes <= lim;
  }
  if (groups > 0x7fffffff) return fail(MI_ERR_UNSUPPORTED, "mi_reshape_and_cache: too many tokens");
  hipStream_t s = as_stream(stream);
  for (int l0 = 0; l0 < num_layers; l0 += kMaxLayersPerLaunch) {
    const int nl = num_layers - l0 < kMaxLayersPerLaunch ? num_layers - l0 : kMaxLayersPerLaunch;
    for (int l = 0; l < nl; ++l) {
      if (!key_src[l0 + l] || !value_src[l0 + l] || !key_pools[l0 + l] || !value_pools[l0 + l])
        return fail(MI_ERR_INVALID_ARGUMENT, "mi_reshape_and_cache: null pointer for layer %d", l0 + l);
      a.key_src[l] = static_cast<const char*>(key_src[l0 + l]);
      a.value_src[l] = static_cast<const char*>(value_src[l0 + l]);
      a.key_pool[l] = static_cast<char*>(key_pools[l0 + l]);
      a.value_pool[l] = static_cast<char*>(value_pools[l0 + l]);
    }
    dim3 grid(static_cast<uint32_t>(groups), nl, span_kernel && kSplitKv ? 2 : 1);
    if (span_kernel && narrow && row_contig)
      reshape_and_cache_span<true, true><<<grid, kSpanThreads, 0, s>>>(a);
    else if (span_kernel && narrow)
      reshape_and_cache_span<true, false><<<grid, kSpanThreads, 0, s>>>(a);
    else if (span_kernel && row_contig)
      reshape_and_cache_span<false, true><<<grid, kSpanThreads, 0, s>>>(a);
    else if (span_kernel)
      reshape_and_cache_span<false, false><<<grid, kSpanThreads, 0, s>>>(a);
    else if (piece == 16)
      reshape_and_cache_generic<u32x4><<<grid, kGenericThreads, 0, s>>>(a);
    else if (piece == 4)
      reshape_and_cache_generic<uint32_t><<<grid, kGenericThreads, 0, s>>>(a);
    else
      reshape_and_cache_generic<uint16_t><<<grid, kGenericThreads, 0, s>>>(a);
    int32_t rc = check_launch("mi_reshape_and_cache");
    if (rc != MI_OK) return rc;
  }
  return ok();
}
