// Kernel 1: reshape-and-cache scatter of new K/V rows into pool slots.
//
// Behaviour of PagedKVCachePool.write_prefill (src/mini_infra/worker/paged_kv_cache.py:74-95)
// and of the decode append in Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:282-283),
// as one launch covering every layer instead of an advanced-index gather plus an index_copy_
// per tensor per layer.
//
// Work mapping: a token is one destination K row and one V row of num_kv_heads * head_dim
// elements (2 KiB each for 8 x 128 bf16), contiguous in the pool.  A workgroup of kThreads lanes
// owns kTokensPerGroup consecutive tokens of one layer.
//  * Row kernel (a token's K+V rows are a multiple of 256 16-byte pieces -- the Qwen3 shape):
//    every lane owns fixed pieces of the row pair, so consecutive lanes move consecutive
//    16-byte pieces of one slot row and each wavefront store is a fully coalesced 1 KiB run.
//    The group's (row, position, slot) triples are staged once through LDS (one coalesced
//    read), then kUnroll tokens' loads are issued before their stores.
//  * Generic kernel (any other row size or misaligned strides): flat piece index with
//    element-size pieces; used by small shapes only.
#include "mi_common.h"

// Measured on MI355X (28-layer prefill store, 40k tokens, token-major source rows; three repetitions
// in one process): 2 tokens per workgroup with one load per lane in flight moves 5.85-5.92 TB/s;
// 2 tokens with 2 in flight 5.79-5.83, 4 with 2 5.57-5.75, 4 with 4 5.35-5.63, 8 with 2 or 4
// 5.13-5.50, 16 with 4 5.22-5.51, 1 token 5.37-5.50.  Many small workgroups keep the most
// independent 2 KiB row copies in flight.  Wider workgroups holding several tokens side by side
// (MI_SCATTER_THREADS) measured slower on another machine: 512 lanes x 2 tokens 5.43-5.44 TB/s,
// x 4 tokens 5.84-5.92, 1024 x 4 5.40-5.57, against 6.04-6.09 for 256 x 2.  Narrower ones, three
// repetitions against the read + write copy ceiling of the same process (6.44 TB/s): 128 lanes x 2
// tokens with both in flight 6.14-6.21 TB/s (95-96%), 256 x 2 with one 6.05-6.17, 128 x 1 token
// 5.93-6.09, 64 lanes 5.45-5.75; K and V rows in separate workgroups (128 x 2 with 2 in flight,
// 128 x 4, 256 x 2) 5.48-6.14.  Device-scope streaming stores (store_stream, which the gather and
// the block records use) against a copy ceiling of 6.69 TB/s with the same stores: 6.07-6.22 TB/s
// at 2 tokens per group against 6.14-6.30 with non-temporal stores; 4, 8 or 16 tokens per group
// with either store 5.14-5.76.  Tokens taken in slot order instead of prompt order: no change
// (6.18-6.20 against 6.15-6.28; 99.9% of consecutive tokens already have consecutive slots).
// Groups mapped so that each XCD takes a contiguous run of tokens: 6.06-6.15 against 6.13-6.22.
// Layers interleaved in dispatch order (all layers of a token group together) instead of one
// layer's groups after another: 5.64-5.88 against 6.16-6.23.
#ifndef MI_SCATTER_TOKENS_PER_GROUP
#define MI_SCATTER_TOKENS_PER_GROUP 2
#endif
#ifndef MI_SCATTER_UNROLL
#define MI_SCATTER_UNROLL 2
#endif
#ifndef MI_SCATTER_NT
#define MI_SCATTER_NT 1
#endif

namespace mi {
namespace {

#ifndef MI_SCATTER_THREADS
#define MI_SCATTER_THREADS 128
#endif
constexpr int kThreads = MI_SCATTER_THREADS;
constexpr int kTokensPerGroup = MI_SCATTER_TOKENS_PER_GROUP;
constexpr int kUnroll = MI_SCATTER_UNROLL;
constexpr bool kNt = MI_SCATTER_NT != 0;  // non-temporal source loads and pool stores
constexpr int kGenericUnroll = 8;
constexpr int kGenericTokensPerGroup = 8;

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
  int32_t tokens_per_group;  // row kernel: tokens per workgroup (<= kTokensPerGroup)
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

// Row kernel: 2 * chunks_per_row (16-byte pieces per token) is a multiple of kThreads.
__global__ __launch_bounds__(kThreads) void reshape_and_cache_rows(const ScatterArgs a) {
  __shared__ int64_t s_key[kTokensPerGroup], s_value[kTokensPerGroup], s_slot[kTokensPerGroup];
  const int layer = blockIdx.y;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * a.tokens_per_group;
  const int ntok = static_cast<int>(min(static_cast<int64_t>(a.tokens_per_group), a.num_tokens - tok0));
  if (static_cast<int>(threadIdx.x) < ntok) {
    const TokenRef t = token_ref(a, tok0 + threadIdx.x);
    s_key[threadIdx.x] = t.key_off;
    s_value[threadIdx.x] = t.value_off;
    s_slot[threadIdx.x] = t.slot;
  }
  __syncthreads();

  const char* key_src = a.key_src[layer];
  const char* value_src = a.value_src[layer];
  char* key_pool = a.key_pool[layer];
  char* value_pool = a.value_pool[layer];
  // Lanes per token: all of them when a token has at least kThreads pieces, else one piece each
  // and kThreads / per_token tokens side by side.
  const uint32_t per_token = 2u * a.chunks_per_row;
  const uint32_t lanes = per_token < kThreads ? per_token : kThreads;
  const int side = static_cast<int>(kThreads / lanes);
  const int t_lane = static_cast<int>(threadIdx.x / lanes);
  for (uint32_t c = threadIdx.x % lanes; c < per_token; c += lanes) {
    // Fixed piece of this lane: K or V, head h, 16-byte column j.
    const bool is_value = c >= a.chunks_per_row;
    const uint32_t w = is_value ? c - a.chunks_per_row : c;
    const uint32_t h = w / a.chunks_per_head;
    const uint32_t j = w - h * a.chunks_per_head;
    const char* src = (is_value ? value_src : key_src) + h * (is_value ? a.value_head : a.key_head) + j * 16u;
    char* dst = (is_value ? value_pool : key_pool) + w * 16u;
    const int64_t* s_off = is_value ? s_value : s_key;
    for (int t0 = t_lane; t0 < ntok; t0 += side * kUnroll) {
      u32x4 val[kUnroll];
#pragma unroll
      for (int k = 0; k < kUnroll; ++k) {
        const int t = t0 + k * side;
        if (t < ntok && s_slot[t] >= 0) val[k] = load_vec<kNt>(reinterpret_cast<const u32x4*>(src + s_off[t]));
      }
#pragma unroll
      for (int k = 0; k < kUnroll; ++k) {
        const int t = t0 + k * side;
        if (t < ntok && s_slot[t] >= 0) store_vec<kNt>(reinterpret_cast<u32x4*>(dst + s_slot[t] * a.row_bytes), val[k]);
      }
    }
  }
}

// Generic kernel: flat piece index, any piece size V.
template <typename V>
__global__ __launch_bounds__(kThreads) void reshape_and_cache_generic(const ScatterArgs a) {
  const int layer = blockIdx.y;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * kGenericTokensPerGroup;
  const int64_t ntok = min(static_cast<int64_t>(kGenericTokensPerGroup), a.num_tokens - tok0);
  const uint32_t per_token = 2u * a.chunks_per_row;  // K row then V row
  const uint32_t n_items = static_cast<uint32_t>(ntok) * per_token;

  for (uint32_t base = 0; base < n_items; base += kThreads * kGenericUnroll) {
    V val[kGenericUnroll];
    V* dst[kGenericUnroll];
#pragma unroll
    for (int k = 0; k < kGenericUnroll; ++k) {
      const uint32_t f = base + k * kThreads + threadIdx.x;
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
  if (num_tokens == 0 || num_layers == 0) return ok();
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
  const bool rows_kernel = wide && ((2u * a.chunks_per_row) % kThreads == 0 || kThreads % (2u * a.chunks_per_row) == 0);
  // Few tokens (a decode append) spread one per workgroup over the CUs; many tokens (a prompt)
  // go kTokensPerGroup per workgroup so each lane keeps kUnroll loads in flight.
  int64_t per_group = kGenericTokensPerGroup;
  if (rows_kernel) {
    const int64_t spread = (num_tokens * num_layers + 2047) / 2048;
    per_group = spread < 1 ? 1 : (spread > kTokensPerGroup ? kTokensPerGroup : spread);
  }
  a.tokens_per_group = static_cast<int32_t>(per_group);

  const int64_t groups = (num_tokens + per_group - 1) / per_group;
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
    dim3 grid(static_cast<uint32_t>(groups), nl);
    if (rows_kernel)
      reshape_and_cache_rows<<<grid, kThreads, 0, s>>>(a);
    else if (piece == 16)
      reshape_and_cache_generic<u32x4><<<grid, kThreads, 0, s>>>(a);
    else if (piece == 4)
      reshape_and_cache_generic<uint32_t><<<grid, kThreads, 0, s>>>(a);
    else
      reshape_and_cache_generic<uint16_t><<<grid, kThreads, 0, s>>>(a);
    int32_t rc = check_launch("mi_reshape_and_cache");
    if (rc != MI_OK) return rc;
  }
  return ok();
}
